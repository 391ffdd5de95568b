// fp32 pre phase on split bf16 MFMA operands: the phi image, support checks
// and the launcher of pre_split_kernel (see mhc_pre_split.hpp).
#include "mhc_pre_split.hpp"

namespace mhc {

// packed[((i*NCB + cb)*NU + u)*64 + lane][s], lane = g*16 + col, for
// k = i*C + cb*32 + 8g + s and feature f = 8u + (col & 7):
//   col < 8:  bf16(phi[k, f])                       (p_hi)
//   col >= 8: bf16(phi[k, f] - bf16(phi[k, f]))     (p_lo)
// and zero past C or FD: lane `lane` of the wave reading column block cb of
// stream i finds its MFMA B operand (8 consecutive k of one column) as one
// 16-byte load.
__global__ __launch_bounds__(256) void phi_pack_split_kernel(const void* __restrict__ phi, int dt,
                                                             uint16_t* __restrict__ packed, int C,
                                                             int FD, int NCB, int NU, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int s = (int)(idx & 7);
  const int lane = (int)((idx >> 3) & 63);
  int64_t rest = idx >> 9;
  const int u = (int)(rest % NU);
  rest /= NU;
  const int cb = (int)(rest % NCB);
  const int i = (int)(rest / NCB);
  const int col = lane & 15;
  const int c = cb * kCBlock + (lane >> 4) * 8 + s;
  const int f = 8 * u + (col & 7);
  float v = 0.f;
  if (c < C && f < FD) {
    const float p = ld_any(phi, ((int64_t)i * C + c) * FD + f, dt);
    const float hi = bf16_bits_to_f32(f32_to_bf16_bits(p));
    v = col < 8 ? hi : p - hi;
  }
  packed[idx] = f32_to_bf16_bits(v);
}

int64_t split_packed_bytes(int n, int C, int mode) {
  if (!(n == 1 || n == 2 || n == 4)) return 0;
  if (mode != kFull && mode != kNoHres && mode != kHead) return 0;
  if (mode == kHead && n == 1) return 0;
  if (C <= 0 || C % 8 != 0) return 0;
  const int ncb = (C + kCBlock - 1) / kCBlock;
  if (ncb > kMfmaMaxColBlocks) return 0;  // C <= 1024
  const int nu = (mode_fd(mode, n) + 7) / 8;
  return (int64_t)n * ncb * nu * 1024;
}

bool split_supported(int x_dtype, int phi_dtype, int n, int C, int mode) {
  return x_dtype == kF32 && phi_dtype == kF32 && split_packed_bytes(n, C, mode) > 0;
}

hipError_t launch_phi_pack_split(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                                 hipStream_t s) {
  const int fd = mode_fd(mode, n);
  const int nu = (fd + 7) / 8;
  const int ncb = (C + kCBlock - 1) / kCBlock;
  const int64_t total = (int64_t)n * ncb * nu * 64 * 8;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(phi_pack_split_kernel, dim3((unsigned)blocks), dim3(256), 0, s, phi, phi_dtype,
                     static_cast<uint16_t*>(packed), C, fd, ncb, nu, total);
  return hipGetLastError();
}

template <int N, int MODE, int KB>
hipError_t launch_pre_split_inst(const PreArgs& a, int num_cus, hipStream_t s) {
  const int64_t ntiles = (a.M + kSplitTok - 1) / kSplitTok;
  const int64_t grid = ntiles < num_cus ? ntiles : num_cus;
  hipLaunchKernelGGL((pre_split_kernel<N, MODE, KB>), dim3((unsigned)grid), dim3(kPersistWaves * 64), 0, s,
                     a, ntiles);
  return hipGetLastError();
}

template <int N, int MODE, int... KBS>
hipError_t dispatch_split_kb(const PreArgs& a, int kb, int num_cus, hipStream_t s) {
  hipError_t r = hipErrorInvalidValue;
  bool done = false;
  ((!done && KBS >= kb ? (r = launch_pre_split_inst<N, MODE, KBS>(a, num_cus, s), done = true) : false),
   ...);
  return r;
}

template <int N>
hipError_t dispatch_split_mode(const PreArgs& a, int kb, int num_cus, hipStream_t s) {
  switch (a.mode) {
    case kFull: return dispatch_split_kb<N, kFull, 1, 2, 3, 4>(a, kb, num_cus, s);
    case kNoHres: return dispatch_split_kb<N, kNoHres, 1, 2, 3, 4>(a, kb, num_cus, s);
    case kHead:
      if constexpr (N > 1) return dispatch_split_kb<N, kHead, 1, 2, 3, 4>(a, kb, num_cus, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pre_split(const PreArgs& a, int num_cus, hipStream_t s) {
  const int kb = persist_kb_needed(a.C);
  switch (a.n) {
    case 1: return dispatch_split_mode<1>(a, kb, num_cus, s);
    case 2: return dispatch_split_mode<2>(a, kb, num_cus, s);
    case 4: return dispatch_split_mode<4>(a, kb, num_cus, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mhc
