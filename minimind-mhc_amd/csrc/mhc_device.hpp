// Device-side helpers shared by the mHC kernels (gfx950 / CDNA4 only).
//
// Storage types: fp32, bf16 and fp16 tensors, all arithmetic in fp32.
// bf16 values are handled as raw 16-bit patterns packed two per dword so that
// 128-bit loads and stores move 8 elements at a time.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

enum Dtype : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

__host__ __device__ inline int dtype_bytes(int dt) { return dt == kF32 ? 4 : 2; }

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

struct alignas(16) U32x4 {
  uint32_t v[4];
};

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 pair (lowers to v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  __bf16 x = (__bf16)a;
  __bf16 y = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) |
         ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float a) {
  __bf16 x = (__bf16)a;
  return __builtin_bit_cast(uint16_t, x);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float a) {
  _Float16 x = (_Float16)a;
  return __builtin_bit_cast(uint16_t, x);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// Load element i of a tensor whose dtype is only known at run time.
__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  if (dt == kF32) return static_cast<const float*>(p)[i];
  uint16_t b = static_cast<const uint16_t*>(p)[i];
  return dt == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

__device__ __forceinline__ void st_any(void* p, int64_t i, int dt, float v) {
  if (dt == kF32) {
    static_cast<float*>(p)[i] = v;
  } else {
    static_cast<uint16_t*>(p)[i] = dt == kBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
  }
}

// Value after a round trip through storage type dt (what a store + reload yields).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (dt == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

// -------------------------------------------------------------- scalar maths

// Logistic function written as 1 / (1 + e^-z), the form torch.sigmoid and
// tl.sigmoid evaluate; mul/add are kept unfused so the gates round like the
// reference's separate torch ops.
__device__ __forceinline__ float sigmoid_f(float z) {
  return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-z)));
}

__device__ __forceinline__ float affine_rn(float s, float alpha, float beta) {
  return __fadd_rn(__fmul_rn(s, alpha), beta);
}

// ------------------------------------------------------ lane-group reductions
// Butterfly reductions over xor-partners: every lane of the group ends with the
// bit-identical result, so all lanes of one Sinkhorn row see the same sum.

template <int MASK_LO, int MASK_HI>
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
  for (int m = MASK_LO; m < MASK_HI; m <<= 1) v = __fadd_rn(v, __shfl_xor(v, m, 64));
  return v;
}

template <int MASK_LO, int MASK_HI>
__device__ __forceinline__ float xor_max(float v) {
#pragma unroll
  for (int m = MASK_LO; m < MASK_HI; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Sinkhorn-Knopp projection of one n x n matrix held one element per lane.
// The group is N*N consecutive lanes (N a power of two, N*N <= 64); lane e of
// the group holds element (row = e / N, col = e % N).  Row partners differ in
// the low log2(N) lane bits, column partners in the next log2(N) bits.
//
// Schedule (model/mhc_fused.py:47-56): softmax over each row, + eps, one column
// normalisation, then (iters - 1) x (row, column) normalisations, each dividing
// by (sum + eps).
template <int N>
__device__ __forceinline__ float sinkhorn_lane(float v, int iters, float eps) {
  constexpr int NN = N * N;
  float mx = xor_max<1, N>(v);
  float e = expf(v - mx);
  float s = xor_sum<1, N>(e);
  v = __fadd_rn(__fdiv_rn(e, s), eps);
  float cs = xor_sum<N, NN>(v);
  v = __fdiv_rn(v, __fadd_rn(cs, eps));
  for (int it = 1; it < iters; ++it) {
    float rs = xor_sum<1, N>(v);
    v = __fdiv_rn(v, __fadd_rn(rs, eps));
    cs = xor_sum<N, NN>(v);
    v = __fdiv_rn(v, __fadd_rn(cs, eps));
  }
  return v;
}

}  // namespace mhc
