// Pre phase: MFMA dispatch, phi packing, and the generic VALU kernel.
//
// The generic kernel serves every (dtype, n, C) the MFMA instances do not:
// fp16 streams, mixed stream / phi dtypes, fp32 outside the split kernel's
// shapes (n <= 4, C <= 1024), C % 8 != 0, and the n == 1 MHCHead (plain
// RMSNorm) at C > 1024.  One 256-thread workgroup per token; it is a
// correctness path, not a tuned one.  x_norm = x * inv_rms is rounded to the
// stream dtype and the projection accumulates in fp32; the gates and the
// pre-aggregate round where the reference's torch ops round
// (model/mhc_fused.py:843-859, model/mhc_fused_no_hres.py:364-386,
// model/mhc_common.py:298-308).
#include "mhc_pre_group.hpp"

namespace mhc {

// ------------------------------------------------------------------ packing

// packed[((i*NCB + cb)*NT + nt)*64 + lane][s] =
//     phi[i*C + cb*32 + (lane/16)*8 + s, nt*16 + lane%16]   (0 outside [C, FD))
// so that lane `lane` of the wave reading column block cb of stream i finds its
// MFMA B operand (8 consecutive k for output column lane%16) as one 16-byte load.
// lo: the image of phi - bf16(phi) instead (the low half of an fp32 phi split
// into bf16 hi + lo operands for the fp32 K-streamed kernel).
__global__ __launch_bounds__(256) void phi_pack_kernel(const void* __restrict__ phi, int dt,
                                                       uint16_t* __restrict__ packed, int C,
                                                       int FD, int NCB, int NT, int64_t total,
                                                       int lo) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int s = (int)(idx & 7);
  const int lane = (int)((idx >> 3) & 63);
  int64_t rest = idx >> 9;
  const int nt = (int)(rest % NT);
  rest /= NT;
  const int cb = (int)(rest % NCB);
  const int i = (int)(rest / NCB);
  const int c = cb * kCBlock + (lane >> 4) * 8 + s;
  const int f = nt * 16 + (lane & 15);
  float v = 0.f;
  if (c < C && f < FD) v = ld_any(phi, ((int64_t)i * C + c) * FD + f, dt);
  const uint16_t hi = f32_to_bf16_bits(v);
  packed[idx] = lo ? f32_to_bf16_bits(v - bf16_bits_to_f32(hi)) : hi;
}

// MFMA kernels: n in {1, 2, 4, 8} at C <= 1024 (register-resident phi for
// n <= 4, the K-streamed kernel for n = 8), and the K-streamed kernel for
// n in {2, 4, 8, 16} at any wider C.  The image is addressed with 32-bit
// byte offsets.
int64_t mfma_packed_bytes(int n, int C, int mode) {
  if (!(n == 1 || n == 2 || n == 4 || n == 8 || n == 16)) return 0;
  if (mode != kFull && mode != kNoHres && mode != kHead) return 0;
  if (mode == kHead && n == 1) return 0;
  if (C <= 0 || C % 8 != 0) return 0;
  const int ncb = (C + kCBlock - 1) / kCBlock;
  if (n == 1 && ncb > kMfmaMaxColBlocks) return 0;  // C <= 1024
  const int fd = mode_fd(mode, n);
  const int nt = (fd + 15) / 16;
  const int64_t bytes = (int64_t)n * ncb * nt * 64 * 8 * 2;
  return bytes <= 0x7fffffffLL ? bytes : 0;
}

// Shapes that take the K-streamed kernel at every batch size.
static bool pre_wide(int n, int C) {
  return n == 16 || (C + kCBlock - 1) / kCBlock > kMfmaMaxColBlocks;
}

bool mfma_supported(int x_dtype, int phi_dtype, int n, int C, int mode) {
  return x_dtype == kBF16 && phi_dtype == kBF16 && mfma_packed_bytes(n, C, mode) > 0;
}

hipError_t launch_phi_pack(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                           hipStream_t s, int lo) {
  const int fd = mode_fd(mode, n);
  const int nt = (fd + 15) / 16;
  const int ncb = (C + kCBlock - 1) / kCBlock;
  const int64_t total = (int64_t)n * ncb * nt * 64 * 8;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(phi_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, s, phi, phi_dtype,
                     static_cast<uint16_t*>(packed), C, fd, ncb, nt, total, lo);
  return hipGetLastError();
}

// fp32 stream and phi on the K-streamed kernel: n = 8 at any C and n in {2, 4}
// past C = 1024 (narrower fp32 rows at n <= 4 take the split kernel).  Its
// image is the packed bf16 layout of bf16(phi) followed by that of
// phi - bf16(phi).
int64_t ks32_packed_bytes(int n, int C, int mode) {
  if (!(n == 8 || ((n == 2 || n == 4) && (C + kCBlock - 1) / kCBlock > kMfmaMaxColBlocks))) return 0;
  const int64_t one = mfma_packed_bytes(n, C, mode);
  return one > 0 && 2 * one <= 0x7fffffffLL ? 2 * one : 0;
}

bool ks32_supported(int x_dtype, int phi_dtype, int n, int C, int mode) {
  return x_dtype == kF32 && phi_dtype == kF32 && ks32_packed_bytes(n, C, mode) > 0;
}

hipError_t launch_phi_pack_ks32(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                                hipStream_t s) {
  const hipError_t e = launch_phi_pack(phi, phi_dtype, packed, n, C, mode, s, 0);
  if (e != hipSuccess) return e;
  return launch_phi_pack(phi, phi_dtype, static_cast<unsigned char*>(packed) + mfma_packed_bytes(n, C, mode),
                         n, C, mode, s, 1);
}

hipError_t launch_pre_kstream_f32(const PreArgs& a, hipStream_t s) {
  switch (a.n) {
    case 2: return launch_pre_kstream_n2(a, s);
    case 4: return launch_pre_kstream_n4(a, s);
    case 8: return launch_pre_kstream_n8(a, s);
    default: return hipErrorInvalidValue;
  }
}

// ------------------------------------------------------ process-wide settings

namespace {
// Batch size up to which the small-batch group kernel runs.  Measured on
// MI355X at C = 768 (pre launch, four rotating input sets): it is ahead of the
// large-batch kernels up to 1024 tokens for n = 2, 4 and 8 (n = 4: 9.7 vs
// 11.0 us at 1024, 7.2 vs 9.7 us at 64; n = 8: 24.9 vs 47.3 us at 1024) and
// level with them at 2048.
int64_t g_token_max_m = 1024;
bool g_row_staging = true;
// Batch size up to which the n = 8 small-batch pre phase runs as two launches
// (projection split over the output tiles, then the rest).
int64_t g_group_split_m = 128;
}  // namespace

int64_t pre_token_max_m() { return g_token_max_m; }
void set_pre_token_max_m(int64_t m) { g_token_max_m = m; }
bool pre_row_staging() { return g_row_staging; }
void set_pre_row_staging(bool on) { g_row_staging = on; }
int64_t pre_group_split_tokens() { return g_group_split_m; }
void set_pre_group_split_tokens(int64_t m) { g_group_split_m = m; }

// Compute units of the current device (cached; one persistent workgroup each).
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev >= 0 && dev < 64 && cache[dev] > 0) return cache[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (dev >= 0 && dev < 64) cache[dev] = cus;
  return cus;
}

hipError_t launch_pre_mfma(const PreArgs& a, hipStream_t s) {
  const int cus = device_cus();
  // n = 16, C > 1024: phi streams from L2 through the K-split MFMA loop.
  if (pre_wide(a.n, a.C)) {
    switch (a.n) {
      case 2: return launch_pre_kstream_n2(a, s);
      case 4: return launch_pre_kstream_n4(a, s);
      case 8: return launch_pre_kstream_n8(a, s);
      case 16: return launch_pre_kstream_n16(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  // Decode-size batches: one workgroup per group of up to 16 tokens.
  if (a.M <= pre_token_max_m() && a.phi_packed) {
    switch (a.n) {
      case 1: return launch_pre_group_n1(a, cus, s);
      case 2: return launch_pre_group_n2(a, cus, s);
      case 4: return launch_pre_group_n4(a, cus, s);
      case 8: return launch_pre_group_n8(a, cus, s);
      default: break;
    }
  }
  // n <= 4: persistent workgroups with the x tile double-buffered in registers.
  if (a.n <= 4) {
    const int kb = persist_kb_needed(a.C);
    switch (a.n) {
      case 1: return launch_pre_persist_n1(a, kb, cus, s);
      case 2: return launch_pre_persist_n2(a, kb, cus, s);
      case 4: return launch_pre_persist_n4(a, kb, cus, s);
      default: break;
    }
  }
  // n = 8: phi (983 KB at C = 768) streams from L2 through a K-split MFMA loop.
  if (a.n == 8) return launch_pre_kstream_n8(a, s);
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------ generic kernel

constexpr int kGenThreads = 256;
constexpr int kGenMaxN = 16;
constexpr int kGenMaxFD = 2 * kGenMaxN + kGenMaxN * kGenMaxN;
constexpr int kGenChunk = 16;  // features reduced per block-wide reduction

// 1 / sqrt(mean_c(v(c)^2) + norm_eps) over the C outputs of this token's
// workgroup (red: kGenThreads / 64 floats of LDS; ends with a barrier).
template <typename F>
__device__ float block_norm_scale(const PreArgs& a, F v, float* red, int tid) {
  float q = 0.f;
  for (int c = tid; c < a.C; c += kGenThreads) {
    const float o = v(c);
    q = fmaf(o, o, q);
  }
  q = wave_sum(q);
  __syncthreads();  // red may hold an earlier reduction's values
  if ((tid & 63) == 0) red[tid >> 6] = q;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < kGenThreads / 64; ++w) t += red[w];
  return 1.0f / sqrtf(t / (float)a.C + a.norm_eps);
}

__global__ __launch_bounds__(kGenThreads) void pre_generic_kernel(PreArgs a) {
  __shared__ float s_red[kGenThreads / 64][kGenChunk];
  __shared__ float s_mix[kGenMaxFD];
  __shared__ float s_hpre[kGenMaxN];
  __shared__ float s_mat[kGenMaxN * kGenMaxN];
  __shared__ float s_inv;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t tok = blockIdx.x;
  const int n = a.n;
  const int C = a.C;
  const int mode = a.mode;
  const int FD = mode_fd(mode, n);
  const int64_t NC = (int64_t)n * C;
  const int xdt = a.x_dtype;
  const int64_t xb = tok * NC;

  // sum of squares over the whole n*C row
  float ss = 0.f;
  for (int64_t k = tid; k < NC; k += kGenThreads) {
    const float v = ld_any(a.x, xb + k, xdt);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if (lane == 0) s_red[wave][0] = ss;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < kGenThreads / 64; ++w) t += s_red[w][0];
    const float inv = 1.0f / sqrtf(t / (float)NC + a.rms_eps);
    s_inv = inv;
    if (a.inv_rms) a.inv_rms[tok] = inv;
  }
  __syncthreads();
  const float inv = s_inv;

  if (mode == kRms) {  // MHCHead with n == 1 (model/mhc_common.py:438-442)
    if (a.norm_w) {
      // the head output rounded to the stream dtype, then the model's final
      // RMSNorm over C (== NC here)
      const float r = block_norm_scale(a, [&](int c) { return round_to(ld_any(a.x, xb + c, xdt) * inv, xdt); },
                                       s_red[0], tid);
      for (int c = tid; c < C; c += kGenThreads)
        st_any(a.sub_in, tok * C + c, xdt,
               round_to(ld_any(a.x, xb + c, xdt) * inv, xdt) * r * ld_any(a.norm_w, c, a.norm_dtype));
      return;
    }
    for (int64_t k = tid; k < NC; k += kGenThreads)
      st_any(a.sub_in, tok * NC + k, xdt, ld_any(a.x, xb + k, xdt) * inv);
    return;
  }

  // projection, kGenChunk output features per block reduction
  for (int f0 = 0; f0 < FD; f0 += kGenChunk) {
    float p[kGenChunk];
#pragma unroll
    for (int j = 0; j < kGenChunk; ++j) p[j] = 0.f;
    for (int64_t k = tid; k < NC; k += kGenThreads) {
      // x_norm rounded to the stream dtype (model/mhc_fused.py:845)
      const float xn = round_to(ld_any(a.x, xb + k, xdt) * inv, xdt);
      const int64_t wb = k * FD + f0;
#pragma unroll
      for (int j = 0; j < kGenChunk; ++j)
        if (f0 + j < FD) p[j] = fmaf(xn, ld_any(a.phi, wb + j, a.phi_dtype), p[j]);
    }
    __syncthreads();  // s_red reuse
#pragma unroll
    for (int j = 0; j < kGenChunk; ++j) {
      const float v = wave_sum(p[j]);
      if (lane == 0) s_red[wave][j] = v;
    }
    __syncthreads();
    if (tid < kGenChunk && f0 + tid < FD) {
      float t = 0.f;
      for (int w = 0; w < kGenThreads / 64; ++w) t += s_red[w][tid];
      s_mix[f0 + tid] = t;
      if (a.mixes_raw) a.mixes_raw[tok * FD + f0 + tid] = t;
    }
  }
  __syncthreads();

  // gates
  const int pdt = a.param_dtype;
  for (int f = tid; f < FD; f += kGenThreads) {
    const float m = s_mix[f];
    if (f < n) {
      const float h = gate_pre(m, ld_any(a.alpha[0], 0, pdt), ld_any(a.bias[0], f, pdt), a.pre_eps, xdt);
      s_hpre[f] = h;
      if (a.h_pre) st_any(a.h_pre, tok * n + f, xdt, h);
    } else if (f < 2 * n) {
      const float h = gate_post(m, ld_any(a.alpha[1], 0, pdt), ld_any(a.bias[1], f - n, pdt),
                                a.post_mult, xdt);
      st_any(a.h_post, tok * n + (f - n), xdt, h);
    } else {
      const int e = f - 2 * n;
      const float h = gate_res(m, ld_any(a.alpha[2], 0, pdt), ld_any(a.bias[2], e, pdt), xdt);
      s_mat[e] = h;
      if (a.h_res_raw) st_any(a.h_res_raw, tok * n * n + e, xdt, h);
    }
  }
  __syncthreads();

  // Sinkhorn-Knopp (model/mhc_fused.py:47-56): thread i owns row i / column i.
  if (mode == kFull && a.h_res) {
    const float eps = a.sk_eps;
    if (tid < n) {
      float* row = s_mat + tid * n;
      float mx = row[0];
      for (int j = 1; j < n; ++j) mx = fmaxf(mx, row[j]);
      float s = 0.f;
      for (int j = 0; j < n; ++j) {
        row[j] = expf(row[j] - mx);
        s += row[j];
      }
      for (int j = 0; j < n; ++j) row[j] = __fadd_rn(__fdiv_rn(row[j], s), eps);
    }
    __syncthreads();
    for (int it = 0; it < a.sk_iters || it == 0; ++it) {
      if (it > 0) {
        if (tid < n) {
          float* row = s_mat + tid * n;
          float s = 0.f;
          for (int j = 0; j < n; ++j) s += row[j];
          const float d = __fadd_rn(s, eps);
          for (int j = 0; j < n; ++j) row[j] = __fdiv_rn(row[j], d);
        }
        __syncthreads();
      }
      if (tid < n) {
        float s = 0.f;
        for (int i = 0; i < n; ++i) s += s_mat[i * n + tid];
        const float d = __fadd_rn(s, eps);
        for (int i = 0; i < n; ++i) s_mat[i * n + tid] = __fdiv_rn(s_mat[i * n + tid], d);
      }
      __syncthreads();
    }
    for (int e = tid; e < n * n; e += kGenThreads) st_any(a.h_res, tok * n * n + e, xdt, s_mat[e]);
  }

  // pre-aggregate (or the MHCHead weighted reduce): each h_pre[i] * x_i product
  // rounds to the stream dtype, the sum over streams accumulates in fp32
  // (model/mhc_fused.py:859, model/mhc_common.py:308).
  auto agg = [&](int c) {
    float o = 0.f;
    for (int i = 0; i < n; ++i)
      o += round_to(s_hpre[i] * ld_any(a.x, xb + (int64_t)i * C + c, xdt), xdt);
    return round_to(o, xdt);
  };
  if (a.norm_w) {  // RMSNorm over C of the rounded pre-aggregate (second pass recomputes it)
    const float r = block_norm_scale(a, agg, s_red[0], tid);
    for (int c = tid; c < C; c += kGenThreads)
      st_any(a.sub_in, tok * C + c, xdt, agg(c) * r * ld_any(a.norm_w, c, a.norm_dtype));
    return;
  }
  for (int c = tid; c < C; c += kGenThreads) st_any(a.sub_in, tok * C + c, xdt, agg(c));
}

hipError_t launch_pre_generic(const PreArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(pre_generic_kernel, dim3((unsigned)a.M), dim3(kGenThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace mhc
