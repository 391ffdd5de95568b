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
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

struct alignas(16) U32x4 {
  uint32_t v[4];
};

// ------------------------------------------------------------ buffer access
// Raw buffer loads/stores bounded by a descriptor's byte count: an offset past
// the end reads zeros / drops the write in hardware.  Masking through the
// descriptor instead of a branch keeps every lane's load unconditional, so the
// compiler can count outstanding loads exactly (s_waitcnt vmcnt(N) rather than
// vmcnt(0)) and prefetched data stays in flight.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kBufDword3 = 0x00020000;   // raw buffer, gfx9-family dword 3
constexpr uint32_t kBufOob = 0x7FFFFFF0u; // an offset past any descriptor used here

// ok ? off : kBufOob, as arithmetic.  Written as a ternary on a per-lane
// condition, the compiler may branch and put the load in both arms; the second
// arm's load into the same registers then waits for every load in flight.
__device__ __forceinline__ uint32_t oob_unless(bool ok, uint32_t off) {
  const uint32_t m = 0u - (uint32_t)ok;
  return (off & m) | (kBufOob & ~m);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kBufDword3);
}

// A wave-uniform 64-bit value pinned to scalar registers.  Where the compiler
// has also materialised a value in vector registers (per-lane addresses built
// from it), a descriptor made from that copy costs a readfirstlane loop around
// every buffer op; the caller asserts uniformity instead.
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Cache policy for data a launch streams exactly once (x in, outputs out): the
// non-temporal bit.  With it the forward's x reads and stream-sized writes
// stop displacing, and being displaced by, the previous launch's dirty lines;
// measured on MI355X at 16384 tokens, n = 4, C = 768 (pre + post step, four
// rotating input sets): 74.5 -> 65.5 us.
constexpr int kNt = 2;
// The same with the device-scope bit (sc1) as well: measured faster for the
// persistent n <= 4 pre kernel (29.9 -> 29.0 us at C2) and slightly slower for
// the n = 8 kernel and the weight kernel, which keep kNt.
constexpr int kNtSc1 = kNt | 16;

template <int POL = kNt>
__device__ __forceinline__ U32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, int soff) {
  return __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, soff, POL));
}

template <int POL = kNt>
__device__ __forceinline__ void buf_store16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, const U32x4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)off, 0, POL);
}

// The same policy through a flat pointer (16 bytes, 16-byte aligned).
__device__ __forceinline__ U32x4 ld16_nt(const void* p) {
  return __builtin_bit_cast(U32x4, __builtin_nontemporal_load(static_cast<const u32x4_t*>(p)));
}

__device__ __forceinline__ void st16_nt(void* p, const U32x4& v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), static_cast<u32x4_t*>(p));
}

__device__ __forceinline__ U32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// 8 / 4 bytes at off into the first dwords of a 16-byte value, the rest zero.
__device__ __forceinline__ U32x4 buf_load8z(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned int u32x2_v __attribute__((ext_vector_type(2)));
  const u32x2_v v = __builtin_bit_cast(u32x2_v, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
  return U32x4{{v.x, v.y, 0u, 0u}};
}
__device__ __forceinline__ U32x4 buf_load4z(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return U32x4{{__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0), 0u, 0u, 0u}};
}

__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, const U32x4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)off, 0, 0);
}

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 pair: one v_cvt_pk_bf16_f32 on gfx950.
// (Two scalar (__bf16) conversions joined by shifts compile to two
// v_cvt_pk_bf16_f32 with a zero operand, a shift and an SDWA or.)
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
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
// A rounded multiply the compiler may not fuse with a later add into an fma.
// HIP's __fmul_rn is the plain operator, which -ffp-contract=fast-honor-pragmas
// (hipcc's default) contracts; the pragma clears the contract flag on this
// multiply only.
__device__ __forceinline__ float mul_nc(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  if (dt == kF32) return static_cast<const float*>(p)[i];
  uint16_t b = static_cast<const uint16_t*>(p)[i];
  return dt == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Raw bits of element i of a tensor whose dtype is only known at run time
// (fp32 bits, or the 16-bit value zero-extended), and the value they hold.
// ld_any converts inside its per-dtype branch, right after the load, so each
// ld_any waits for its own load before the next one issues; raw loads carry no
// conversion, so a kernel can put all of its loads in flight first.
__device__ __forceinline__ uint32_t ld_raw(const void* p, int64_t i, int dt) {
  if (dt == kF32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float raw_to_f32(uint32_t b, int dt) {
  if (dt == kF32) return __builtin_bit_cast(float, b);
  return dt == kBF16 ? bf16_bits_to_f32((uint16_t)b) : f16_bits_to_f32((uint16_t)b);
}

// Element q (0..3) of four consecutive elements loaded as one 16-byte buffer
// word group (buf_load16 at the first element's byte offset): fp32 takes word
// q, a 16-bit dtype the half q & 1 of word q >> 1.  One unconditional load per
// lane instead of a per-dtype branch around each element.
__device__ __forceinline__ float word4_elem(const U32x4& w, int q, int dt) {
  if (dt == kF32) return __builtin_bit_cast(float, w.v[q]);
  const uint32_t h = (q & 1) ? w.v[q >> 1] >> 16 : w.v[q >> 1] & 0xffffu;
  return dt == kBF16 ? bf16_bits_to_f32((uint16_t)h) : f16_bits_to_f32((uint16_t)h);
}
// Element i of a run-time-dtype tensor from the 4-byte word that holds it (a
// 16-bit element's word starts at (2i) & ~3; for tensors of an even count of
// 16-bit elements that word lies inside the tensor).
__device__ __forceinline__ uint32_t word_off(int64_t i, int dt) {
  return dt == kF32 ? (uint32_t)i * 4u : ((uint32_t)i * 2u) & ~3u;
}
__device__ __forceinline__ float word_elem(uint32_t w, int64_t i, int dt) {
  if (dt == kF32) return __builtin_bit_cast(float, w);
  const uint32_t h = (i & 1) ? w >> 16 : w & 0xffffu;
  return dt == kBF16 ? bf16_bits_to_f32((uint16_t)h) : f16_bits_to_f32((uint16_t)h);
}

// The 4-byte word holding element i of a run-time-dtype vector of `count`
// elements (count even for a 16-bit dtype), through a buffer descriptor: one
// unconditional load and no per-dtype branch, so later loads do not wait for
// it; word_elem converts it where the value is first needed.
__device__ __forceinline__ uint32_t ld_word(const void* p, int64_t count, int64_t i, int dt) {
  const uint32_t bytes = (uint32_t)count * (dt == kF32 ? 4u : 2u);
  return buf_load4z(make_rsrc(p, bytes), word_off(i, dt)).v[0];
}

// Bits of element i of a run-time-dtype tensor of `count` elements (0 when
// !ok or p is null), with no branch: two 2-byte buffer loads, the element's
// low and high halves for fp32, and for a 16-bit dtype the element and an
// out-of-range offset (reads zero, touches no memory).  Every byte read lies
// inside the tensor, and with no per-dtype branch later loads do not wait for
// these; bits_to_f32 converts where the value is needed.
__device__ __forceinline__ uint32_t ld_bits(const void* p, int64_t count, int64_t i, int dt, bool ok) {
  const bool f32 = dt == kF32;
  const auto r = make_rsrc(p, p ? (uint32_t)count * (f32 ? 4u : 2u) : 0u);
  const uint32_t lo = ok ? (uint32_t)i * (f32 ? 4u : 2u) : kBufOob;
  const uint32_t hi = ok && f32 ? (uint32_t)i * 4u + 2u : kBufOob;
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)lo, 0, 0) |
         ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)hi, 0, 0) << 16);
}
__device__ __forceinline__ float bits_to_f32(uint32_t b, int dt) {
  if (dt == kF32) return __builtin_bit_cast(float, b);
  return dt == kBF16 ? bf16_bits_to_f32((uint16_t)b) : f16_bits_to_f32((uint16_t)b);
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
  return __fadd_rn(mul_nc(s, alpha), beta);
}

// ---------------------------------------------- reference rounding points
// The reference's PyTorch path evaluates the gates as separate torch ops on
// tensors of the stream dtype (model/mhc_fused.py:846-854): the projection
// output mixes is a stream-dtype tensor, then (m * alpha), (+ bias),
// sigmoid, and (+ pre_eps) / (* post_mult) each round to that dtype.  These
// helpers apply the same roundings (all no-ops for fp32 streams).

// sigmoid(alpha * m + bias) with the reference's roundings.
__device__ __forceinline__ float gate_sigmoid(float m, float alpha, float bias, int dt) {
  const float mq = round_to(m, dt);
  const float z = round_to(__fadd_rn(round_to(mul_nc(mq, alpha), dt), bias), dt);
  return round_to(sigmoid_f(z), dt);
}

// h_pre (and the MHCHead mix): sigmoid(...) + pre_eps
__device__ __forceinline__ float gate_pre(float m, float alpha, float bias, float pre_eps, int dt) {
  return round_to(__fadd_rn(gate_sigmoid(m, alpha, bias, dt), pre_eps), dt);
}

// h_post: sigmoid(...) * post_mult
__device__ __forceinline__ float gate_post(float m, float alpha, float bias, float post_mult, int dt) {
  return round_to(mul_nc(gate_sigmoid(m, alpha, bias, dt), post_mult), dt);
}

// h_res_raw: alpha * m + bias (Sinkhorn then runs in fp32 on this value)
__device__ __forceinline__ float gate_res(float m, float alpha, float bias, int dt) {
  return round_to(__fadd_rn(round_to(mul_nc(round_to(m, dt), alpha), dt), bias), dt);
}

// ------------------------------------------------------- x_norm on packed bf16
// bf16(x * inv) for the 8 columns of one 16-byte chunk: the fp32 product
// rounded to bf16, as the reference's x_norm = (x.float() * inv_rms).to(x.dtype)
// (model/mhc_fused.py:845) rounds it.
__device__ __forceinline__ U32x4 x_norm_chunk(const U32x4& v, float inv) {
  U32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) o.v[j] = pack_bf16x2(bf16lo(v.v[j]) * inv, bf16hi(v.v[j]) * inv);
  return o;
}

// ------------------------------------------- pre-aggregate on packed bf16
// sub_in[c] = bf16( sum_i bf16(h_i * x_i[c]) ) for one 16-byte chunk (8
// columns) of each of the N streams, with the reference's rounding points
// (model/mhc_fused.py:859: each product is a bf16 tensor element, the sum over
// streams accumulates in fp32).  v_dot2c_f32_bf16 forms each product exactly
// from the packed pair (h_i is bf16, so h_i * x is exact in fp32) with no
// unpacking: (x_lo, x_hi) . (h, 0) and (x_lo, x_hi) . (0, h).  Two streams'
// rounded products share one packed register and one dot2 with (1, 1) adds
// both into the fp32 sum.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// One packed column pair: x[i] holds columns (c, c + 1) of stream i.
template <int N>
__device__ __forceinline__ uint32_t preagg_pair(const uint32_t (&x)[N], const uint32_t (&hlo)[N],
                                                const uint32_t (&hhi)[N]) {
  constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 (1.0, 1.0)
  float plo[N];
  float phi_[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    plo[i] = dot2_bf16(x[i], hlo[i], 0.f);
    phi_[i] = dot2_bf16(x[i], hhi[i], 0.f);
  }
  float slo;
  float shi;
  if constexpr (N == 1) {
    slo = plo[0];
    shi = phi_[0];
  } else {
    slo = 0.f;
    shi = 0.f;
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      slo = dot2_bf16(pack_bf16x2(plo[i], plo[i + 1]), kOnes, slo);
      shi = dot2_bf16(pack_bf16x2(phi_[i], phi_[i + 1]), kOnes, shi);
    }
  }
  return pack_bf16x2(slo, shi);
}

template <int N>
__device__ __forceinline__ U32x4 preagg_chunk(const U32x4 (&x)[N], const uint32_t (&hlo)[N],
                                             const uint32_t (&hhi)[N]) {
  U32x4 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t xj[N];
#pragma unroll
    for (int i = 0; i < N; ++i) xj[i] = x[i].v[j];
    out.v[j] = preagg_pair<N>(xj, hlo, hhi);
  }
  return out;
}

// (h, 0) and (0, h) packed bf16 pairs for preagg_chunk; h must be bf16-exact.
__device__ __forceinline__ uint32_t pack_lo(float h) { return (uint32_t)f32_to_bf16_bits(h); }
__device__ __forceinline__ uint32_t pack_hi(float h) { return (uint32_t)f32_to_bf16_bits(h) << 16; }

// ------------------------------------------------------ lane-group reductions
// Sinkhorn keeps one matrix element per lane; row and column sums are
// butterflies over lane groups.  Within 16-lane rows they use DPP (fused into
// v_add_f32_dpp): quad_perm for lane xor 1 / 2, row_ror:8 for xor 8, and
// row_ror:4 / row_half_mirror for xor 4 once the value is already symmetric
// under xor 8 / within quads (so every lane of a group ends with the
// bit-identical sum).  Partners 16 and 32 lanes apart use ds_swizzle/bpermute.

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, true));
}

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124;       // row_ror:4
constexpr int kDppRor8 = 0x128;       // row_ror:8  (== lane xor 8 inside a row)
constexpr int kDppHalfMirror = 0x141; // row_half_mirror (lane i <-> 7-i in each 8)
constexpr int kDppRowMirror = 0x140;  // row_mirror (lane i <-> 15-i in each 16)

struct OpAdd {
  __device__ static float f(float a, float b) { return a + b; }
};
struct OpMax {
  __device__ static float f(float a, float b) { return fmaxf(a, b); }
};

// Reduce over the N consecutive lanes of one matrix row (N in {1, 2, 4, 8}).
template <int N, typename Op>
__device__ __forceinline__ float row_reduce(float v) {
  if constexpr (N >= 2) v = Op::f(v, dpp_f<kDppXor1>(v));
  if constexpr (N >= 4) v = Op::f(v, dpp_f<kDppXor2>(v));
  if constexpr (N >= 8) v = Op::f(v, dpp_f<kDppHalfMirror>(v));
  return v;
}

// The value of the lane 16 (32) lanes away: v_permlane16_swap /
// v_permlane32_swap exchange rows of two registers without going through LDS.
// Fed two copies of v, the first result holds v of the even rows (halves) and
// the second of the odd ones, so each lane's partner value is whichever of
// the two is not its own.  The copy goes through an opaque move: given the
// same value twice the compiler folds the two results into one.
__device__ __forceinline__ float xor_lane16(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v);
  uint32_t b;
  asm volatile("v_mov_b32 %0, %1" : "=v"(b) : "v"(a));
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  const bool odd_row = (__lane_id() >> 4) & 1;
  return __builtin_bit_cast(float, odd_row ? r[0] : r[1]);
}
__device__ __forceinline__ float xor_lane32(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v);
  uint32_t b;
  asm volatile("v_mov_b32 %0, %1" : "=v"(b) : "v"(a));
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  const bool upper = __lane_id() >= 32;
  return __builtin_bit_cast(float, upper ? r[0] : r[1]);
}

// Sum over the 16 lanes of a DPP row (both halves, then the mirror): every
// lane of the row ends with the bit-identical total.
__device__ __forceinline__ float row16_sum(float v) {
  v = row_reduce<8, OpAdd>(v);
  return v + dpp_f<kDppRowMirror>(v);
}

// Sum over all 64 lanes of the wave; every lane ends with the bit-identical
// total (each step adds a value and its partner's, a commutative pair).
__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_f<kDppXor1>(v);
  v = v + dpp_f<kDppXor2>(v);
  v = v + dpp_f<kDppHalfMirror>(v);
  v = v + dpp_f<kDppRowMirror>(v);
  v = v + xor_lane16(v);
  v = v + xor_lane32(v);
  return v;
}

// Reduce over the N lanes of one matrix column (stride N inside N*N lanes).
template <int N>
__device__ __forceinline__ float col_sum(float v) {
  if constexpr (N == 2) {
    v = v + dpp_f<kDppXor2>(v);
  } else if constexpr (N == 4) {
    v = v + dpp_f<kDppRor8>(v);
    v = v + dpp_f<kDppRor4>(v);
  } else if constexpr (N == 8) {
    v = v + dpp_f<kDppRor8>(v);
    v = v + xor_lane16(v);
    v = v + xor_lane32(v);
  }
  return v;
}

// Sinkhorn-Knopp projection of one n x n matrix held one element per lane.
// The group is N*N consecutive lanes (N a power of two, N*N <= 64); lane e of
// the group holds element (row = e / N, col = e % N).
//
// Schedule (model/mhc_fused.py:47-56): softmax over each row, + eps, one column
// normalisation, then (iters - 1) x (row, column) normalisations, each dividing
// by (sum + eps).  Divisions use the hardware reciprocal (<= 1 ulp) and a
// multiply; sums are fp32 butterflies.
template <int N>
__device__ __forceinline__ float sinkhorn_lane(float v, int iters, float eps) {
  const float mx = row_reduce<N, OpMax>(v);
  const float e = expf(v - mx);
  const float s = row_reduce<N, OpAdd>(e);
  v = e * __builtin_amdgcn_rcpf(s) + eps;
  v = v * __builtin_amdgcn_rcpf(col_sum<N>(v) + eps);
  for (int it = 1; it < iters; ++it) {
    v = v * __builtin_amdgcn_rcpf(row_reduce<N, OpAdd>(v) + eps);
    v = v * __builtin_amdgcn_rcpf(col_sum<N>(v) + eps);
  }
  return v;
}

// ------------------------------------------ 8 x 8 Sinkhorn, half a row per lane
// One matrix per 16 lanes: lane j of the group holds row (j & 7), columns
// 4 * (j >> 3) .. + 3 in v[0..3].  A row sum is three in-lane adds and one DPP
// add with the lane 8 away (the row's other half; the sum is commutative, so
// both halves get the bit-identical value).  A column sum is the 8-lane
// butterfly of row_reduce over the lanes of one half (rows 0..7).  Lane j
// forms the reciprocal of only column (j & 3) of its half (its quad position)
// and quad_perm broadcasts hand each lane the four it needs, so a column
// step costs one v_rcp per lane instead of four.  The schedule and the
// (sum + eps) divisors are those of sinkhorn_lane<8>; only the order of the
// fp32 additions inside a sum differs.

__device__ __forceinline__ float sk8_row_sum(const float (&v)[4]) {
  const float s = (v[0] + v[1]) + (v[2] + v[3]);
  return s + dpp_f<kDppRor8>(s);
}

__device__ __forceinline__ void sk8_row_norm(float (&v)[4], float eps) {
  const float r = __builtin_amdgcn_rcpf(sk8_row_sum(v) + eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = v[q] * r;
}

__device__ __forceinline__ void sk8_col_norm(float (&v)[4], float eps) {
  float c[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) c[q] = row_reduce<8, OpAdd>(v[q]);
  const int l = __lane_id();
  const float lo = (l & 1) ? c[1] : c[0];
  const float hi = (l & 1) ? c[3] : c[2];
  const float r = __builtin_amdgcn_rcpf(((l & 2) ? hi : lo) + eps);
  v[0] = v[0] * dpp_f<0x00>(r);  // quad_perm [0,0,0,0]
  v[1] = v[1] * dpp_f<0x55>(r);  // quad_perm [1,1,1,1]
  v[2] = v[2] * dpp_f<0xAA>(r);  // quad_perm [2,2,2,2]
  v[3] = v[3] * dpp_f<0xFF>(r);  // quad_perm [3,3,3,3]
}

// Softmax over each row, + eps, then the first column normalisation.
__device__ __forceinline__ void sk8_start(float (&v)[4], float eps) {
  float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
  mx = fmaxf(mx, dpp_f<kDppRor8>(mx));
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = expf(v[q] - mx);
  const float r = __builtin_amdgcn_rcpf(sk8_row_sum(v));
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = v[q] * r + eps;
  sk8_col_norm(v, eps);
}

// One of the remaining (iters - 1) row + column normalisations.
__device__ __forceinline__ void sk8_iter(float (&v)[4], float eps) {
  sk8_row_norm(v, eps);
  sk8_col_norm(v, eps);
}

// ---------------------------------------- 16 x 16 Sinkhorn, half a row per lane
// One matrix per 32 lanes (two DPP rows): lane j of the group holds row
// (j >> 1), columns 8 * (j & 1) .. + 7 in v[0..7].  A row sum is seven in-lane
// adds and one DPP add with the neighbouring lane (the row's other half).  A
// column sum runs over the 16 lanes of one parity (j & 1): lane xor 2
// (quad_perm), xor 8 (row_ror:8), then row_ror:4, which adds lane j + 4 or its
// xor-8 partner (the value is already symmetric under xor 8), and the other
// DPP row (lane xor 16); each step adds two bit-identical values, so every
// lane of a column ends with the bit-identical sum.  Schedule and (sum + eps)
// divisors as sinkhorn_lane.

__device__ __forceinline__ float sk16_row_sum(const float (&v)[8]) {
  const float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  return s + dpp_f<kDppXor1>(s);
}

__device__ __forceinline__ float sk16_col_sum(float c) {
  c = c + dpp_f<kDppXor2>(c);
  c = c + dpp_f<kDppRor8>(c);
  c = c + dpp_f<kDppRor4>(c);
  return c + xor_lane16(c);
}

__device__ __forceinline__ void sk16_col_norm(float (&v)[8], float eps) {
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = v[q] * __builtin_amdgcn_rcpf(sk16_col_sum(v[q]) + eps);
}

__device__ __forceinline__ void sk16_start(float (&v)[8], float eps) {
  float mx = fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
  mx = fmaxf(mx, dpp_f<kDppXor1>(mx));
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = expf(v[q] - mx);
  const float r = __builtin_amdgcn_rcpf(sk16_row_sum(v));
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = v[q] * r + eps;
  sk16_col_norm(v, eps);
}

__device__ __forceinline__ void sk16_iter(float (&v)[8], float eps) {
  const float r = __builtin_amdgcn_rcpf(sk16_row_sum(v) + eps);
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = v[q] * r;
  sk16_col_norm(v, eps);
}

}  // namespace mhc
