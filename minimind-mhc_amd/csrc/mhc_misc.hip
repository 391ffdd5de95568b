// Standalone Sinkhorn-Knopp (sinkhorn_normalize) and StreamExpand.
#include "mhc_internal.hpp"

namespace mhc {

// ------------------------------------------------------------- Sinkhorn-Knopp
// Batched n x n projection onto the doubly-stochastic set, fp32 arithmetic,
// output in the input dtype (model/mhc_fused.py:61-93, :111-128; schedule
// :47-56).  n in {1, 2, 4, 8}: one element per lane, lane-group shuffles.

template <int N>
__global__ __launch_bounds__(256) void sinkhorn_lane_kernel(const void* __restrict__ in,
                                                            void* __restrict__ out, int dt,
                                                            int64_t total, int iters, float eps) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool ok = e < total;  // total is a multiple of N*N, and 256 % (N*N) == 0
  float v = ok ? ld_any(in, e, dt) : 0.f;
  v = sinkhorn_lane<N>(v, iters, eps);
  if (ok) st_any(out, e, dt, v);
}

// Any n <= 32: one workgroup per matrix, thread i owns row i / column i, the
// matrix lives in LDS.
constexpr int kSkMaxN = 32;

__global__ __launch_bounds__(64) void sinkhorn_lds_kernel(const void* __restrict__ in,
                                                          void* __restrict__ out, int dt, int n,
                                                          int iters, float eps) {
  __shared__ float s[kSkMaxN * kSkMaxN];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * n * n;
  for (int e = tid; e < n * n; e += 64) s[e] = ld_any(in, base + e, dt);
  __syncthreads();
  if (tid < n) {
    float* row = s + tid * n;
    float mx = row[0];
    for (int j = 1; j < n; ++j) mx = fmaxf(mx, row[j]);
    float sum = 0.f;
    for (int j = 0; j < n; ++j) {
      row[j] = expf(row[j] - mx);
      sum += row[j];
    }
    for (int j = 0; j < n; ++j) row[j] = __fadd_rn(__fdiv_rn(row[j], sum), eps);
  }
  __syncthreads();
  for (int it = 0; it < iters || it == 0; ++it) {
    if (it > 0) {
      if (tid < n) {
        float* row = s + tid * n;
        float sum = 0.f;
        for (int j = 0; j < n; ++j) sum += row[j];
        const float d = __fadd_rn(sum, eps);
        for (int j = 0; j < n; ++j) row[j] = __fdiv_rn(row[j], d);
      }
      __syncthreads();
    }
    if (tid < n) {
      float sum = 0.f;
      for (int i = 0; i < n; ++i) sum += s[i * n + tid];
      const float d = __fadd_rn(sum, eps);
      for (int i = 0; i < n; ++i) s[i * n + tid] = __fdiv_rn(s[i * n + tid], d);
    }
    __syncthreads();
  }
  for (int e = tid; e < n * n; e += 64) st_any(out, base + e, dt, s[e]);
}

hipError_t launch_sinkhorn(const void* in, void* out, int dtype, int64_t batch, int n, int iters,
                           float eps, hipStream_t s) {
  const int64_t total = batch * n * n;
  const int64_t blocks = (total + 255) / 256;
  switch (n) {
    case 1:
      hipLaunchKernelGGL(sinkhorn_lane_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, dtype, total, iters, eps);
      break;
    case 2:
      hipLaunchKernelGGL(sinkhorn_lane_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, dtype, total, iters, eps);
      break;
    case 4:
      hipLaunchKernelGGL(sinkhorn_lane_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, dtype, total, iters, eps);
      break;
    case 8:
      hipLaunchKernelGGL(sinkhorn_lane_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, dtype, total, iters, eps);
      break;
    default:
      if (n > kSkMaxN) return hipErrorInvalidValue;
      hipLaunchKernelGGL(sinkhorn_lds_kernel, dim3((unsigned)batch), dim3(64), 0, s, in, out, dtype, n, iters, eps);
      break;
  }
  return hipGetLastError();
}

// --------------------------------------------------------------- StreamExpand
// out[t, i*C + c] = x[t, c] for i < n (model/mhc_common.py:115-119); a pure
// byte copy, so it is written over units of U (16, 4 or 2 bytes).

template <typename U>
__global__ __launch_bounds__(256) void expand_kernel(const U* __restrict__ x, U* __restrict__ out,
                                                     int64_t total, int n, int cu) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= total) return;
  const int64_t per_tok = (int64_t)n * cu;
  const int64_t tok = gid / per_tok;
  const int c = (int)((gid - tok * per_tok) % cu);
  out[gid] = x[tok * cu + c];
}

hipError_t launch_stream_expand(const void* x, void* out, int elem_bytes, int64_t M, int n, int C,
                                hipStream_t s) {
  const int64_t row_bytes = (int64_t)elem_bytes * C;
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out);
  if (row_bytes % 16 == 0 && align % 16 == 0) {
    const int cu = (int)(row_bytes / 16);
    const int64_t total = M * n * cu;
    hipLaunchKernelGGL(expand_kernel<U32x4>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       static_cast<const U32x4*>(x), static_cast<U32x4*>(out), total, n, cu);
  } else if (row_bytes % 4 == 0 && align % 4 == 0) {
    const int cu = (int)(row_bytes / 4);
    const int64_t total = M * n * cu;
    hipLaunchKernelGGL(expand_kernel<uint32_t>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint32_t*>(x), static_cast<uint32_t*>(out), total, n, cu);
  } else {
    const int cu = (int)(row_bytes / 2);
    const int64_t total = M * n * cu;
    hipLaunchKernelGGL(expand_kernel<uint16_t>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), total, n, cu);
  }
  return hipGetLastError();
}

// ------------------------------------------------- RMSNorm + StreamExpand
// The model's entry (model/model_minimind.py:365): RMSNorm(C) with gain w,
// then n copies (model/mhc_common.py:115-119), in one pass:
//   y[c] = round(x[c] * (1 / sqrt(mean_c(x^2) + eps)) * w[c]),  out[t, i*C + c] = y[c].
// One wave per token; fp32 arithmetic, one rounding to the stream dtype.
// With n = 1 it is a plain RMSNorm, also in place (out == x): each lane
// reads its chunks of the row before it writes them.

__device__ __forceinline__ float lo16(uint32_t u, int dt) {
  return dt == kBF16 ? bf16lo(u) : f16_bits_to_f32((uint16_t)(u & 0xffffu));
}
__device__ __forceinline__ float hi16(uint32_t u, int dt) {
  return dt == kBF16 ? bf16hi(u) : f16_bits_to_f32((uint16_t)(u >> 16));
}
__device__ __forceinline__ uint32_t pack16(float a, float b, int dt) {
  if (dt == kBF16) return pack_bf16x2(a, b);
  return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

// 16-bit streams, C % 8 == 0, 16-byte aligned rows: 8 elements per lane step.
// out_ssq (optional, bf16, C % 128 == 0): the sum of the squares of the
// written row (n times that of one normed copy) in out_ssq[token][0], the
// token's other C / 128 - 1 partials zero (see PreArgs::x_ssq).
__global__ __launch_bounds__(256) void expand_norm_vec_kernel(const U32x4* x, int xdt,
                                                              const void* __restrict__ w, int wdt,
                                                              U32x4* out, int64_t M,
                                                              int n, int C, float eps,
                                                              float* __restrict__ out_ssq) {
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= M) return;  // whole waves
  const int lane = threadIdx.x & 63;
  const int C8 = C >> 3;
  const U32x4* xr = x + tok * C8;
  float ss = 0.f;
  for (int ch = lane; ch < C8; ch += 64) {
    const U32x4 v = xr[ch];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = lo16(v.v[j], xdt);
      const float b = hi16(v.v[j], xdt);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)C + eps);
  U32x4* orow = out + tok * n * C8;
  float q = 0.f;
  for (int ch = lane; ch < C8; ch += 64) {
    const U32x4 v = xr[ch];
    U32x4 y;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = ch * 8 + 2 * j;
      y.v[j] = pack16(lo16(v.v[j], xdt) * r * ld_any(w, c, wdt),
                      hi16(v.v[j], xdt) * r * ld_any(w, c + 1, wdt), xdt);
    }
    for (int i = 0; i < n; ++i) orow[(int64_t)i * C8 + ch] = y;
    if (out_ssq) {  // uniform
#pragma unroll
      for (int j = 0; j < 4; ++j) q = dot2_bf16(y.v[j], y.v[j], q);
    }
  }
  if (out_ssq) {  // uniform
    q = wave_sum(q) * (float)n;
    const int P = C / kSsqCols;
    for (int j = lane; j < P; j += 64) out_ssq[tok * P + j] = j == 0 ? q : 0.f;
  }
}

__global__ __launch_bounds__(256) void expand_norm_kernel(const void* x, int xdt,
                                                          const void* __restrict__ w, int wdt,
                                                          void* out, int64_t M, int n,
                                                          int C, float eps) {
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= M) return;
  const int lane = threadIdx.x & 63;
  const int64_t xb = tok * C;
  float ss = 0.f;
  for (int c = lane; c < C; c += 64) {
    const float v = ld_any(x, xb + c, xdt);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)C + eps);
  const int64_t ob = tok * n * C;
  for (int c = lane; c < C; c += 64) {
    const float y = ld_any(x, xb + c, xdt) * r * ld_any(w, c, wdt);
    for (int i = 0; i < n; ++i) st_any(out, ob + (int64_t)i * C + c, xdt, y);
  }
}

hipError_t launch_expand_norm(const void* x, int x_dtype, const void* w, int w_dtype, void* out,
                              int64_t M, int n, int C, float eps, hipStream_t s, float* out_ssq) {
  const unsigned blocks = (unsigned)((M + 3) / 4);
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out);
  if (x_dtype != kF32 && C % 8 == 0 && align % 16 == 0) {
    if (out_ssq && !ssq_supported(x_dtype, C)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(expand_norm_vec_kernel, dim3(blocks), dim3(256), 0, s,
                       static_cast<const U32x4*>(x), x_dtype, w, w_dtype, static_cast<U32x4*>(out),
                       M, n, C, eps, out_ssq);
  } else {
    if (out_ssq) return hipErrorInvalidValue;  // sums of squares: the vector kernel only
    hipLaunchKernelGGL(expand_norm_kernel, dim3(blocks), dim3(256), 0, s, x, x_dtype, w, w_dtype,
                       out, M, n, C, eps);
  }
  return hipGetLastError();
}

}  // namespace mhc
