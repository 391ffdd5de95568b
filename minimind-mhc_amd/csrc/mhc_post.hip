// Post phase: res-mix + post-expand, one read-n / write-n streaming pass.
//
//   out[t, i, c] = sum_j H_res[t, i, j] * x[t, j, c] + H_post[t, i] * F[t, c]
//   (use_mhc = 2, H_res = I:  out[t, i, c] = x[t, i, c] + H_post[t, i] * F[t, c])
//
// Reference: model/mhc_fused.py:416-459 (fused kernel), :562-568 (ref),
// model/mhc_fused_no_hres.py:284-316, :389-394.  fp32 arithmetic, one rounding
// at each point where the reference's torch ops round (see post_vec_kernel).
//
// Work split: one thread per (token, V-column chunk), V = 16 bytes of x.  The
// thread reads the n chunks of x at that column, the F chunk, and the token's
// n*n + n gate values (broadcast within the token's threads), and writes n
// chunks of out.  Every byte of x, F and out moves exactly once.
#include <type_traits>

#include "mhc_internal.hpp"

namespace mhc {

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  __device__ static float get(float v) { return v; }
  __device__ static float put(float v) { return v; }
};
template <>
struct Elem<__bf16> {
  __device__ static float get(__bf16 v) { return bf16_bits_to_f32(__builtin_bit_cast(uint16_t, v)); }
  __device__ static __bf16 put(float v) { return (__bf16)v; }
};
template <>
struct Elem<_Float16> {
  __device__ static float get(_Float16 v) { return (float)v; }
  __device__ static _Float16 put(float v) { return (_Float16)v; }
};

// K contiguous elements moved as one aligned aggregate (K * sizeof(T) is a power
// of two, so the compiler emits the widest vector load/store that fits).
template <typename T, int K>
struct alignas(K * sizeof(T) >= 16 ? 16 : K * sizeof(T)) Pack {
  T v[K];
};

template <typename T, int K>
__device__ __forceinline__ void load_pack(const T* p, float (&o)[K]) {
  const Pack<T, K> pk = *reinterpret_cast<const Pack<T, K>*>(p);
#pragma unroll
  for (int k = 0; k < K; ++k) o[k] = Elem<T>::get(pk.v[k]);
}

// 16-byte packs with the non-temporal cache policy (data streamed once).
template <typename T, int K>
__device__ __forceinline__ void load_pack_nt(const T* p, float (&o)[K]) {
  static_assert(sizeof(Pack<T, K>) == 16, "16-byte packs");
  const Pack<T, K> pk =
      __builtin_bit_cast(Pack<T, K>, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
#pragma unroll
  for (int k = 0; k < K; ++k) o[k] = Elem<T>::get(pk.v[k]);
}

template <typename T, int K>
__device__ __forceinline__ void store_pack_nt(T* p, const float (&o)[K]) {
  static_assert(sizeof(Pack<T, K>) == 16, "16-byte packs");
  Pack<T, K> pk;
#pragma unroll
  for (int k = 0; k < K; ++k) pk.v[k] = Elem<T>::put(o[k]);
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, pk), reinterpret_cast<u32x4_t*>(p));
}

template <typename T, int K>
__device__ __forceinline__ void store_pack(T* p, const float (&o)[K]) {
  Pack<T, K> pk;
#pragma unroll
  for (int k = 0; k < K; ++k) pk.v[k] = Elem<T>::put(o[k]);
  *reinterpret_cast<Pack<T, K>*>(p) = pk;
}

// Value after a store to / reload from element type T.
template <typename T>
__device__ __forceinline__ float rnd(float v) {
  return Elem<T>::get(Elem<T>::put(v));
}

// Rounding points follow the reference's torch ops (model/mhc_fused.py:861-863):
// the einsum result, the H_post * F product and their sum are each a tensor of
// the stream dtype.  x reads and out writes are non-temporal (each byte once per
// launch); F keeps the default policy (measured slower non-temporal).
// SSQ (bf16 streams, C % 128 == 0): each DPP row of 16 threads covers 128
// columns of one token (C / 8 threads a token, a multiple of 16, rows aligned
// to tokens); its sum of the squares of the stored outputs over every stream
// goes to out_ssq[token][column / 128], the sums of squares the next pre
// launch would otherwise form with a pass over the row of its own.
template <typename XT, typename FT, int N, bool RES, bool SSQ>
__global__ __launch_bounds__(256) void post_vec_kernel(PostArgs a) {
  constexpr int V = 16 / sizeof(XT);
  static_assert(!SSQ || std::is_same_v<XT, __bf16>, "sums of squares for bf16 streams");
  const int C = a.C;
  const int CV = C / V;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t tok = gid / CV;
  if (tok >= a.M) return;
  const int c = (int)(gid - tok * CV) * V;
  const int64_t NC = (int64_t)N * C;
  const XT* __restrict__ x = static_cast<const XT*>(a.x) + tok * NC + c;
  XT* __restrict__ out = static_cast<XT*>(a.out) + tok * NC + c;

  float xv[N][V];
#pragma unroll
  for (int j = 0; j < N; ++j) load_pack_nt<XT, V>(x + (int64_t)j * C, xv[j]);
  float fv[V];
  load_pack<FT, V>(static_cast<const FT*>(a.f_out) + tok * C + c, fv);
  float hp[N];
  load_pack<XT, N>(static_cast<const XT*>(a.h_post) + tok * N, hp);
  float hr[RES ? N * N : 1];
  if constexpr (RES) load_pack<XT, N * N>(static_cast<const XT*>(a.h_res) + tok * N * N, hr);

  float q = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float o[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float acc;
      if constexpr (RES) {
        acc = 0.f;
#pragma unroll
        for (int j = 0; j < N; ++j) acc = fmaf(hr[i * N + j], xv[j][v], acc);
        acc = rnd<XT>(acc);
      } else {
        acc = xv[i][v];
      }
      o[v] = __fadd_rn(acc, rnd<XT>(mul_nc(hp[i], fv[v])));
    }
    if constexpr (SSQ) {  // the stored pairs, squared on dot2 (exact products, fp32 sum)
      u32x4_t ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = pack_bf16x2(o[2 * e], o[2 * e + 1]);
      __builtin_nontemporal_store(ov, reinterpret_cast<u32x4_t*>(out + (int64_t)i * C));
#pragma unroll
      for (int e = 0; e < 4; ++e) q = dot2_bf16(ov[e], ov[e], q);
    } else {
      store_pack_nt<XT, V>(out + (int64_t)i * C, o);
    }
  }
  if constexpr (SSQ) {
    q = row16_sum(q);
    const int ch = (int)(gid - tok * CV);
    if ((ch & 15) == 0) a.out_ssq[tok * (CV / 16) + (ch >> 4)] = q;
  }
}

// n = 16, bf16 stream, gates and F.  post_vec_kernel's one thread per column
// chunk would hold 256 gate values a thread; here one wave takes a token and
// its lanes stride over 4-column chunks (8 bytes of each stream).  The gates
// are wave-uniform and come through the scalar cache, h_res one row at a time
// as bf16 pairs of adjacent streams (h_res[i][2p], h_res[i][2p+1]): the
// row-major layout already pairs them.  The x chunk is re-packed once into the
// matching pairs (x[2p][c], x[2p+1][c]) by v_perm, and each res-mix output is
// eight v_dot2_f32_bf16 (bf16 products are exact in fp32; the fp32 sum runs
// pairwise rather than in post_vec_kernel's order).  Rounding points as
// post_vec_kernel.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// SSQ: the wave's sum of the squares of the token's stored outputs goes to
// out_ssq[token][0], the token's other C / 128 - 1 partials are zero.
template <bool RES, bool SSQ>
__global__ __launch_bounds__(256) void post_n16_kernel(PostArgs a) {
  constexpr int N = 16;
  constexpr int NP = N / 2;
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tok >= a.M) return;  // whole wave
  const int C = a.C;
  const int C4 = C / 4;
  const int64_t NC = (int64_t)N * C;
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(a.x) + tok * NC;
  const uint16_t* __restrict__ f = static_cast<const uint16_t*>(a.f_out) + tok * C;
  uint16_t* __restrict__ out = static_cast<uint16_t*>(a.out) + tok * NC;
  const uint32_t* __restrict__ hp32 =
      reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.h_post) + tok * N);
  const uint32_t* __restrict__ hr32 =
      RES ? reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.h_res) + tok * N * N) : nullptr;
  float hp[N];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const uint32_t w = __builtin_amdgcn_readfirstlane(hp32[p]);
    hp[2 * p] = bf16lo(w);
    hp[2 * p + 1] = bf16hi(w);
  }
  float q = 0.f;
  for (int cv = lane; cv < C4; cv += 64) {
    const int c = cv * 4;
    u32x2_t xv[N];
#pragma unroll
    for (int j = 0; j < N; ++j)
      xv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(x + (int64_t)j * C + c));
    const u32x2_t fv = *reinterpret_cast<const u32x2_t*>(f + c);
    const float fl[4] = {bf16lo(fv.x), bf16hi(fv.x), bf16lo(fv.y), bf16hi(fv.y)};
    // xp[p][k] = (x[2p][c + k], x[2p + 1][c + k])
    uint32_t xp[RES ? NP : 1][4];
    if constexpr (RES) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          xp[p][2 * h] = __builtin_amdgcn_perm(xv[2 * p + 1][h], xv[2 * p][h], 0x05040100u);
          xp[p][2 * h + 1] = __builtin_amdgcn_perm(xv[2 * p + 1][h], xv[2 * p][h], 0x07060302u);
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float r[4];
      if constexpr (RES) {
        uint32_t hrow[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) hrow[p] = __builtin_amdgcn_readfirstlane(hr32[i * NP + p]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float acc = 0.f;
#pragma unroll
          for (int p = 0; p < NP; ++p) acc = dot2_bf16(hrow[p], xp[p][k], acc);
          r[k] = rnd<__bf16>(acc);
        }
      } else {
        r[0] = bf16lo(xv[i].x);
        r[1] = bf16hi(xv[i].x);
        r[2] = bf16lo(xv[i].y);
        r[3] = bf16hi(xv[i].y);
      }
      float o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = __fadd_rn(r[k], rnd<__bf16>(mul_nc(hp[i], fl[k])));
      const u32x2_t ov = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      __builtin_nontemporal_store(ov, reinterpret_cast<u32x2_t*>(out + (int64_t)i * C + c));
      if constexpr (SSQ) q = dot2_bf16(ov.y, ov.y, dot2_bf16(ov.x, ov.x, q));
    }
  }
  if constexpr (SSQ) {
    q = wave_sum(q);
    const int P = C / kSsqCols;
    for (int j = lane; j < P; j += 64) a.out_ssq[tok * P + j] = j == 0 ? q : 0.f;
  }
}

// n = 8, bf16 stream, gates and F: post_vec_kernel's split (one thread per
// token and 16-byte column chunk), with x and H_res kept packed.  Unpacked,
// the 64 x values and 64 H_res values of a thread take 116 VGPRs (four waves
// a SIMD).  Here the chunk is re-packed once into stream pairs
// (x[2p][c], x[2p+1][c]) by v_perm and each res-mix output is four
// v_dot2_f32_bf16 against H_res row i's adjacent pairs, as post_n16_kernel
// does (the fp32 sum runs pairwise rather than in post_vec_kernel's order).
// SSQ as post_vec_kernel.
template <bool RES, bool SSQ>
__global__ __launch_bounds__(256) void post_n8_kernel(PostArgs a) {
  constexpr int N = 8;
  constexpr int NP = N / 2;
  const int C = a.C;
  const int CV = C / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t tok = gid / CV;
  if (tok >= a.M) return;
  const int c = (int)(gid - tok * CV) * 8;
  const int64_t NC = (int64_t)N * C;
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(a.x) + tok * NC + c;
  uint16_t* __restrict__ out = static_cast<uint16_t*>(a.out) + tok * NC + c;
  u32x4_t xv[N];
#pragma unroll
  for (int j = 0; j < N; ++j)
    xv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + (int64_t)j * C));
  const u32x4_t fv = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.f_out) + tok * C + c);
  const u32x4_t hpv = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.h_post) + tok * N);
  float fl[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    fl[2 * e] = bf16lo(fv[e]);
    fl[2 * e + 1] = bf16hi(fv[e]);
  }
  u32x4_t hr[RES ? N : 1];  // row i: its four adjacent pairs (h_res[i][2p], h_res[i][2p + 1])
  uint32_t xp[RES ? NP : 1][8];     // xp[p][k] = (x[2p][c + k], x[2p + 1][c + k])
  if constexpr (RES) {
    const u32x4_t* hr4 = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.h_res) + tok * N * N);
#pragma unroll
    for (int i = 0; i < N; ++i) hr[i] = hr4[i];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xp[p][2 * e] = __builtin_amdgcn_perm(xv[2 * p + 1][e], xv[2 * p][e], 0x05040100u);
        xp[p][2 * e + 1] = __builtin_amdgcn_perm(xv[2 * p + 1][e], xv[2 * p][e], 0x07060302u);
      }
  }
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float hp = (i & 1) ? bf16hi(hpv[i >> 1]) : bf16lo(hpv[i >> 1]);
    float o[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float r;
      if constexpr (RES) {
        float acc = 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) acc = dot2_bf16(hr[i][p], xp[p][k], acc);
        r = rnd<__bf16>(acc);
      } else {
        r = (k & 1) ? bf16hi(xv[i][k >> 1]) : bf16lo(xv[i][k >> 1]);
      }
      o[k] = __fadd_rn(r, rnd<__bf16>(mul_nc(hp, fl[k])));
    }
    u32x4_t ov;
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = pack_bf16x2(o[2 * e], o[2 * e + 1]);
    __builtin_nontemporal_store(ov, reinterpret_cast<u32x4_t*>(out + (int64_t)i * C));
    if constexpr (SSQ) {  // squares of the stored pairs, exact products, fp32 sum
#pragma unroll
      for (int e = 0; e < 4; ++e) q = dot2_bf16(ov[e], ov[e], q);
    }
  }
  if constexpr (SSQ) {
    q = row16_sum(q);
    const int ch = (int)(gid - tok * CV);
    if ((ch & 15) == 0) a.out_ssq[tok * (CV / 16) + (ch >> 4)] = q;
  }
}

// Any dtype mix, any C: one thread per output element.
__global__ __launch_bounds__(256) void post_generic_kernel(PostArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int n = a.n;
  const int C = a.C;
  const int64_t per_tok = (int64_t)n * C;
  const int64_t tok = gid / per_tok;
  if (tok >= a.M) return;
  const int64_t rem = gid - tok * per_tok;
  const int i = (int)(rem / C);
  const int c = (int)(rem - (int64_t)i * C);
  const int64_t xb = tok * per_tok;
  const int xdt = a.x_dtype;
  float acc;
  if (a.h_res) {
    acc = 0.f;
    for (int j = 0; j < n; ++j)
      acc = fmaf(ld_any(a.h_res, tok * n * n + i * n + j, a.h_dtype),
                 ld_any(a.x, xb + (int64_t)j * C + c, xdt), acc);
    acc = round_to(acc, xdt);
  } else {
    acc = ld_any(a.x, xb + (int64_t)i * C + c, xdt);
  }
  const float wb = round_to(mul_nc(ld_any(a.h_post, tok * n + i, a.h_dtype),
                                      ld_any(a.f_out, tok * C + c, a.f_dtype)), xdt);
  st_any(a.out, xb + (int64_t)i * C + c, xdt, __fadd_rn(acc, wb));
}

template <typename XT, typename FT, int N>
static hipError_t launch_vec(const PostArgs& a, hipStream_t s) {
  constexpr int V = 16 / sizeof(XT);
  const int64_t threads = a.M * (a.C / V);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if constexpr (std::is_same_v<XT, __bf16> && N <= 4) {
    if (a.out_ssq) {
      if (a.h_res)
        hipLaunchKernelGGL((post_vec_kernel<XT, FT, N, true, true>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((post_vec_kernel<XT, FT, N, false, true>), grid, dim3(256), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.out_ssq) return hipErrorInvalidValue;  // no sums-of-squares form of this kernel
  if (a.h_res)
    hipLaunchKernelGGL((post_vec_kernel<XT, FT, N, true, false>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((post_vec_kernel<XT, FT, N, false, false>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <typename XT, typename FT>
static hipError_t launch_vec_n(const PostArgs& a, hipStream_t s) {
  switch (a.n) {
    case 1: return launch_vec<XT, FT, 1>(a, s);
    case 2: return launch_vec<XT, FT, 2>(a, s);
    case 4: return launch_vec<XT, FT, 4>(a, s);
    case 8: return launch_vec<XT, FT, 8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipError_t launch_post(const PostArgs& a, hipStream_t s) {
  const int xb = dtype_bytes(a.x_dtype);
  const int V = 16 / xb;
  // n == 16 would hold 256 gate values per thread: one wave per token instead.
  if (a.n == 16 && a.x_dtype == kBF16 && a.h_dtype == kBF16 && a.f_dtype == kBF16 && a.C % 4 == 0 &&
      ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.out) |
        reinterpret_cast<uintptr_t>(a.f_out)) & 7) == 0 &&
      ((reinterpret_cast<uintptr_t>(a.h_post) | reinterpret_cast<uintptr_t>(a.h_res)) & 3) == 0) {
    const dim3 grid((unsigned)((a.M + 3) / 4));
    if (a.out_ssq) {
      if (a.h_res)
        hipLaunchKernelGGL((post_n16_kernel<true, true>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((post_n16_kernel<false, true>), grid, dim3(256), 0, s, a);
    } else {
      if (a.h_res)
        hipLaunchKernelGGL((post_n16_kernel<true, false>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((post_n16_kernel<false, false>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
  }
  if (a.n == 8 && a.x_dtype == kBF16 && a.h_dtype == kBF16 && a.f_dtype == kBF16 && a.C % 8 == 0 &&
      aligned16(a.x) && aligned16(a.out) && aligned16(a.f_out) && aligned16(a.h_post) &&
      (!a.h_res || aligned16(a.h_res))) {
    const dim3 grid((unsigned)((a.M * (a.C / 8) + 255) / 256));
    if (a.out_ssq) {
      if (a.h_res)
        hipLaunchKernelGGL((post_n8_kernel<true, true>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((post_n8_kernel<false, true>), grid, dim3(256), 0, s, a);
    } else {
      if (a.h_res)
        hipLaunchKernelGGL((post_n8_kernel<true, false>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((post_n8_kernel<false, false>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
  }
  const bool pow2n = a.n == 1 || a.n == 2 || a.n == 4 || a.n == 8;
  const bool vec_ok = pow2n && a.h_dtype == a.x_dtype && a.C % V == 0 && aligned16(a.x) &&
                      aligned16(a.out) && aligned16(a.f_out) &&
                      (reinterpret_cast<uintptr_t>(a.h_post) % (a.n * xb > 16 ? 16 : a.n * xb)) == 0 &&
                      (!a.h_res ||
                       (reinterpret_cast<uintptr_t>(a.h_res) % (a.n * a.n * xb > 16 ? 16 : a.n * a.n * xb)) == 0);
  if (vec_ok) {
    if (a.x_dtype == kBF16 && a.f_dtype == kBF16) return launch_vec_n<__bf16, __bf16>(a, s);
    if (a.x_dtype == kF32 && a.f_dtype == kF32) return launch_vec_n<float, float>(a, s);
    // fp32 stream, bf16 F: the reference trainers' autocast layout.
    if (a.x_dtype == kF32 && a.f_dtype == kBF16) return launch_vec_n<float, __bf16>(a, s);
    if (a.x_dtype == kF16 && a.f_dtype == kF16) return launch_vec_n<_Float16, _Float16>(a, s);
  }
  if (a.out_ssq) return hipErrorInvalidValue;  // sums of squares: bf16 vector kernels only
  const int64_t total = a.M * a.n * (int64_t)a.C;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(post_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ============================================================ backward
// Per token (model/mhc_fused.py:462-526):
//   g_x[j, c]     = sum_i h_res[i, j] * g[i, c]       (g_x = g without h_res)
//   g_h_res[i, j] = sum_c g[i, c] * x[j, c]
//   g_h_post[i]   = sum_c g[i, c] * F[c]
//   g_F[c]        = sum_i h_post[i] * g[i, c]
// fp32 arithmetic, one rounding at each store (the reference kernel's
// tl.store casts), as one wave per token: lanes stride over the token's
// 16-byte column chunks, then wave_sum reduces the n^2 + n dot products.

template <typename XT, typename FT, int N, bool RES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(N >= 8 ? 2 : 1))) void post_bwd_vec_kernel(PostBwdArgs a) {
  constexpr int V = 16 / sizeof(XT);
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tok >= a.M) return;  // whole wave
  const int C = a.C;
  const int CV = C / V;
  const int64_t NC = (int64_t)N * C;
  const XT* __restrict__ x = static_cast<const XT*>(a.x) + tok * NC;
  const XT* __restrict__ g = static_cast<const XT*>(a.g_out) + tok * NC;
  const FT* __restrict__ f = static_cast<const FT*>(a.f_out) + tok * C;
  XT* __restrict__ gx = a.g_x ? static_cast<XT*>(a.g_x) + tok * NC : nullptr;
  FT* __restrict__ gf = static_cast<FT*>(a.g_f) + tok * C;

  float hp[N];
  load_pack<XT, N>(static_cast<const XT*>(a.h_post) + tok * N, hp);
  float hr[RES ? N * N : 1];
  if constexpr (RES) load_pack<XT, N * N>(static_cast<const XT*>(a.h_res) + tok * N * N, hr);
  float ahr[RES ? N * N : 1];
  float ahp[N];
#pragma unroll
  for (int k = 0; k < (RES ? N * N : 1); ++k) ahr[k] = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) ahp[i] = 0.f;

  for (int cv = lane; cv < CV; cv += 64) {
    const int c = cv * V;
    float gv[N][V];
#pragma unroll
    for (int i = 0; i < N; ++i) load_pack_nt<XT, V>(g + (int64_t)i * C + c, gv[i]);
    float fv[V];
    load_pack<FT, V>(f + c, fv);
    if constexpr (RES) {
      float xv[N][V];
#pragma unroll
      for (int j = 0; j < N; ++j) load_pack_nt<XT, V>(x + (int64_t)j * C + c, xv[j]);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < N; ++i) acc = fmaf(hr[i * N + j], gv[i][v], acc);
          o[v] = acc;
        }
        store_pack_nt<XT, V>(gx + (int64_t)j * C + c, o);
      }
#pragma unroll
      for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < N; ++j)
#pragma unroll
          for (int v = 0; v < V; ++v) ahr[i * N + j] = fmaf(gv[i][v], xv[j][v], ahr[i * N + j]);
    } else if (gx) {
#pragma unroll
      for (int j = 0; j < N; ++j) store_pack_nt<XT, V>(gx + (int64_t)j * C + c, gv[j]);
    }
    float o[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < N; ++i) acc = fmaf(hp[i], gv[i][v], acc);
      o[v] = acc;
    }
    store_pack<FT, V>(gf + c, o);
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int v = 0; v < V; ++v) ahp[i] = fmaf(gv[i][v], fv[v], ahp[i]);
  }
  // Reduce over the wave; lane k stores value k.
  float mine_hr = 0.f;
  if constexpr (RES) {
#pragma unroll
    for (int k = 0; k < N * N; ++k) {
      const float t = wave_sum(ahr[k]);
      mine_hr = lane == k ? t : mine_hr;
    }
  }
  float mine_hp = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float t = wave_sum(ahp[i]);
    mine_hp = lane == i ? t : mine_hp;
  }
  if constexpr (RES) {
    if (lane < N * N) static_cast<XT*>(a.g_h_res)[tok * N * N + lane] = Elem<XT>::put(mine_hr);
  }
  if (lane < N) static_cast<XT*>(a.g_h_post)[tok * N + lane] = Elem<XT>::put(mine_hp);
}

// bf16 streams, n in {2, 4, 8}: the same one-wave-per-token split with
// packed operands.  h_res and h_post are wave-uniform and sit in scalar
// registers as bf16 pairs of adjacent streams, (h[2p][j], h[2p+1][j]); every
// product runs on v_dot2_f32_bf16 (a bf16 x bf16 product is exact in fp32,
// and each dot2 adds two of them to an fp32 accumulator):
//   g_h_res[i][j] += g_i . x_j,  g_h_post[i] += g_i . F   (4 column pairs a chunk)
//   g_x[j][c] = sum_p (h[2p][j], h[2p+1][j]) . (g[2p][c], g[2p+1][c])
//   g_F[c]    = sum_p (hp[2p], hp[2p+1])     . (g[2p][c], g[2p+1][c])
// with the stream pairs of each column built once per chunk by v_perm.  g and
// x stay packed (4 VGPRs per 8 columns, not 8 fp32), so n = 8 fits three
// waves per SIMD with no spills where the fp32 form needed more than 256
// VGPRs.  Sums run in a different order than post_bwd_vec_kernel's fmaf
// chains: results agree to fp32 rounding before the bf16 store.  g and x
// reads and the g_x / g_F writes are non-temporal (68.7 -> 60.5 us at 16384
// tokens, n = 4, C = 768 on MI355X); F keeps the default policy.
template <int N, bool RES>
__global__ __launch_bounds__(256) void post_bwd_bf16_kernel(PostBwdArgs a) {
  static_assert(N % 2 == 0, "pairs of streams");
  constexpr int NP = N / 2;
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tok >= a.M) return;  // whole wave
  const int C = a.C;
  const int CV = C / 8;
  const int64_t NC = (int64_t)N * C;
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(a.x) + tok * NC;
  const uint16_t* __restrict__ g = static_cast<const uint16_t*>(a.g_out) + tok * NC;
  const uint16_t* __restrict__ f = static_cast<const uint16_t*>(a.f_out) + tok * C;
  uint16_t* __restrict__ gx = a.g_x ? static_cast<uint16_t*>(a.g_x) + tok * NC : nullptr;
  uint16_t* __restrict__ gf = static_cast<uint16_t*>(a.g_f) + tok * C;

  // Gate pairs: element (i, j) of the token's row-major gates is half (j & 1)
  // of dword (i * N + j) / 2 (N even).
  const uint32_t* __restrict__ hp32 =
      reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.h_post) + tok * N);
  uint32_t hp2[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) hp2[p] = __builtin_amdgcn_readfirstlane(hp32[p]);
  uint32_t hr2[RES ? NP * N : 1];
  if constexpr (RES) {
    const uint32_t* __restrict__ hr32 =
        reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.h_res) + tok * N * N);
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const uint32_t w0 = hr32[(2 * p * N + j) >> 1];
        const uint32_t w1 = hr32[((2 * p + 1) * N + j) >> 1];
        const uint32_t v = (j & 1) ? ((w0 >> 16) | (w1 & 0xffff0000u)) : ((w0 & 0xffffu) | (w1 << 16));
        hr2[p * N + j] = __builtin_amdgcn_readfirstlane(v);
      }
  }
  float ahr[RES ? N * N : 1];
  float ahp[N];
#pragma unroll
  for (int k = 0; k < (RES ? N * N : 1); ++k) ahr[k] = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) ahp[i] = 0.f;

  for (int cv = lane; cv < CV; cv += 64) {
    const int c = cv * 8;
    U32x4 gv[N];
#pragma unroll
    for (int i = 0; i < N; ++i) gv[i] = ld16_nt(g + (int64_t)i * C + c);
    const U32x4 fv = *reinterpret_cast<const U32x4*>(f + c);
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) ahp[i] = dot2_bf16(gv[i].v[k], fv.v[k], ahp[i]);
    if constexpr (RES) {
      U32x4 xv[N];
#pragma unroll
      for (int j = 0; j < N; ++j) xv[j] = ld16_nt(x + (int64_t)j * C + c);
#pragma unroll
      for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < N; ++j)
#pragma unroll
          for (int k = 0; k < 4; ++k) ahr[i * N + j] = dot2_bf16(gv[i].v[k], xv[j].v[k], ahr[i * N + j]);
    } else if (gx) {
#pragma unroll
      for (int j = 0; j < N; ++j) *reinterpret_cast<U32x4*>(gx + (int64_t)j * C + c) = gv[j];
    }
    // (g[2p][c], g[2p+1][c]) for the low (even) and high (odd) column of each pair k
    uint32_t glo[NP][4];
    uint32_t ghi[NP][4];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        glo[p][k] = __builtin_amdgcn_perm(gv[2 * p + 1].v[k], gv[2 * p].v[k], 0x05040100u);
        ghi[p][k] = __builtin_amdgcn_perm(gv[2 * p + 1].v[k], gv[2 * p].v[k], 0x07060302u);
      }
    U32x4 of;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float lo = 0.f;
      float hi = 0.f;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        lo = dot2_bf16(hp2[p], glo[p][k], lo);
        hi = dot2_bf16(hp2[p], ghi[p][k], hi);
      }
      of.v[k] = pack_bf16x2(lo, hi);
    }
    st16_nt(gf + c, of);
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < N; ++j) {
        U32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float lo = 0.f;
          float hi = 0.f;
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            lo = dot2_bf16(hr2[p * N + j], glo[p][k], lo);
            hi = dot2_bf16(hr2[p * N + j], ghi[p][k], hi);
          }
          o.v[k] = pack_bf16x2(lo, hi);
        }
        if (gx) st16_nt(gx + (int64_t)j * C + c, o);
      }
    }
  }
  // Reduce over the wave; lane k stores value k.
  float mine_hr = 0.f;
  if constexpr (RES) {
#pragma unroll
    for (int k = 0; k < N * N; ++k) {
      const float t = wave_sum(ahr[k]);
      mine_hr = lane == k ? t : mine_hr;
    }
  }
  float mine_hp = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float t = wave_sum(ahp[i]);
    mine_hp = lane == i ? t : mine_hp;
  }
  if constexpr (RES) {
    if (lane < N * N) static_cast<__bf16*>(a.g_h_res)[tok * N * N + lane] = (__bf16)mine_hr;
  }
  if (lane < N) static_cast<__bf16*>(a.g_h_post)[tok * N + lane] = (__bf16)mine_hp;
}

// Any dtypes, n <= 16, any C: one 256-thread workgroup per token.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is reused by consecutive calls
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void post_bwd_generic_kernel(PostBwdArgs a) {
  __shared__ float red[4];
  const int64_t tok = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = a.n;
  const int C = a.C;
  const int64_t NC = (int64_t)n * C;
  const int64_t xb = tok * NC;
  const int xdt = a.x_dtype, hdt = a.h_dtype, fdt = a.f_dtype;
  const bool res = a.h_res != nullptr;
  if (a.g_x) {
    for (int64_t e = tid; e < NC; e += 256) {
      const int j = (int)(e / C);
      const int c = (int)(e - (int64_t)j * C);
      float acc;
      if (res) {
        acc = 0.f;
        for (int i = 0; i < n; ++i)
          acc = fmaf(ld_any(a.h_res, tok * n * n + i * n + j, hdt),
                     ld_any(a.g_out, xb + (int64_t)i * C + c, xdt), acc);
      } else {
        acc = ld_any(a.g_out, xb + e, xdt);
      }
      st_any(a.g_x, xb + e, xdt, acc);
    }
  }
  for (int c = tid; c < C; c += 256) {
    float acc = 0.f;
    for (int i = 0; i < n; ++i)
      acc = fmaf(ld_any(a.h_post, tok * n + i, hdt), ld_any(a.g_out, xb + (int64_t)i * C + c, xdt), acc);
    st_any(a.g_f, tok * C + c, fdt, acc);
  }
  const int np = (res ? n * n : 0) + n;
  for (int p = 0; p < np; ++p) {  // uniform
    float acc = 0.f;
    if (p < (res ? n * n : 0)) {
      const int i = p / n;
      const int j = p - i * n;
      for (int c = tid; c < C; c += 256)
        acc = fmaf(ld_any(a.g_out, xb + (int64_t)i * C + c, xdt), ld_any(a.x, xb + (int64_t)j * C + c, xdt), acc);
    } else {
      const int i = p - (res ? n * n : 0);
      for (int c = tid; c < C; c += 256)
        acc = fmaf(ld_any(a.g_out, xb + (int64_t)i * C + c, xdt), ld_any(a.f_out, tok * C + c, fdt), acc);
    }
    const float t = block_sum256(acc, red);
    if (tid == 0) {
      if (p < (res ? n * n : 0)) st_any(a.g_h_res, tok * n * n + p, hdt, t);
      else st_any(a.g_h_post, tok * n + (p - (res ? n * n : 0)), hdt, t);
    }
  }
}

template <typename XT, typename FT, int N>
static hipError_t launch_bwd_vec(const PostBwdArgs& a, hipStream_t s) {
  const int64_t blocks = (a.M + 3) / 4;
  if (a.h_res)
    hipLaunchKernelGGL((post_bwd_vec_kernel<XT, FT, N, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((post_bwd_vec_kernel<XT, FT, N, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int N>
static hipError_t launch_bwd_bf16(const PostBwdArgs& a, hipStream_t s) {
  const int64_t blocks = (a.M + 3) / 4;
  if (a.h_res)
    hipLaunchKernelGGL((post_bwd_bf16_kernel<N, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((post_bwd_bf16_kernel<N, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

// bf16: the packed dot2 kernel for paired streams, the fp32 form at n = 1.
static hipError_t launch_bwd_bf16_n(const PostBwdArgs& a, hipStream_t s) {
  switch (a.n) {
    case 1: return launch_bwd_vec<__bf16, __bf16, 1>(a, s);
    case 2: return launch_bwd_bf16<2>(a, s);
    case 4: return launch_bwd_bf16<4>(a, s);
    case 8: return launch_bwd_bf16<8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename XT, typename FT>
static hipError_t launch_bwd_vec_n(const PostBwdArgs& a, hipStream_t s) {
  switch (a.n) {
    case 1: return launch_bwd_vec<XT, FT, 1>(a, s);
    case 2: return launch_bwd_vec<XT, FT, 2>(a, s);
    case 4: return launch_bwd_vec<XT, FT, 4>(a, s);
    case 8: return launch_bwd_vec<XT, FT, 8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_post_bwd(const PostBwdArgs& a, hipStream_t s) {
  const int xb = dtype_bytes(a.x_dtype);
  const int V = 16 / xb;
  const bool pow2n = a.n == 1 || a.n == 2 || a.n == 4 || a.n == 8;
  auto small_ok = [&](const void* p, int elems) {
    const int al = elems * xb > 16 ? 16 : elems * xb;
    return p == nullptr || (reinterpret_cast<uintptr_t>(p) % al) == 0;
  };
  // F in the stream dtype, or bf16 F beside an fp32 stream (autocast training).
  const bool f_ok = a.f_dtype == a.x_dtype || (a.x_dtype == kF32 && a.f_dtype == kBF16);
  const bool vec_ok = pow2n && a.h_dtype == a.x_dtype && f_ok && a.C % V == 0 &&
                      aligned16(a.x) && aligned16(a.g_out) && aligned16(a.f_out) &&
                      aligned16(a.g_f) && (a.g_x == nullptr || aligned16(a.g_x)) &&
                      small_ok(a.h_post, a.n) && small_ok(a.h_res, a.n * a.n);
  if (vec_ok) {
    if (a.x_dtype == kBF16) return launch_bwd_bf16_n(a, s);
    if (a.x_dtype == kF32 && a.f_dtype == kBF16) return launch_bwd_vec_n<float, __bf16>(a, s);
    if (a.x_dtype == kF32) return launch_bwd_vec_n<float, float>(a, s);
    if (a.x_dtype == kF16) return launch_bwd_vec_n<_Float16, _Float16>(a, s);
  }
  hipLaunchKernelGGL(post_bwd_generic_kernel, dim3((unsigned)a.M), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace mhc
