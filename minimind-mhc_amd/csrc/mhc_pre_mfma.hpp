// Fused mHC pre phase on MFMA, bf16 streams (gfx950).
//
// One workgroup owns a tile of 16 tokens (the M side of
// v_mfma_f32_16x16x32_bf16).  The token tile's n*C stream row is split over
// the workgroup's waves by 32-column blocks: wave w owns column blocks
// cb = w, w + WAVES, w + 2*WAVES, ... for every stream i, so it holds
// x[t, i*C + cb*32 .. +32] for all n streams of those columns.  That makes the
// later pre-aggregate (sum over streams at a fixed column) wave-local.
//
// Per token the kernel computes, with x read from HBM exactly once:
//   ss        = sum_k x[k]^2                    (fp32, from the held registers)
//   acc[f]    = sum_k x[k] * phi[k, f]          (MFMA, fp32 accumulate)
//   inv_rms   = 1 / sqrt(ss / (n*C) + rms_eps)
//   mixes[f]  = acc[f] * inv_rms                (== (x * inv_rms) @ phi)
//   gates     h_pre = sigmoid(a_pre*m + b_pre) + pre_eps
//             h_post = 2*sigmoid(a_post*m + b_post)   (post_mult)
//             h_res_raw = a_res*m + b_res
//             each op rounded to bf16 as the reference's torch ops round it
//   h_res     = Sinkhorn(h_res_raw) in fp32     (one matrix element per lane)
//   sub_in[c] = sum_i bf16(h_pre[i] * x[i*C + c])
// Reference semantics: model/mhc_fused.py:163-268 (fused kernel),
// :533-559 (_pre_phase_full_ref), :47-56 (Sinkhorn), :820-830 (module flow);
// model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195 (head).
//
// Register budget: x tile = KB * N * 4 VGPRs per lane (KB column blocks per
// wave, N streams, 16 bytes each).  Instances keep KB * N <= 32.
#pragma once

#include "mhc_internal.hpp"

namespace mhc {

// 4 waves per workgroup, 8 for n >= 8 (keeps the x tile at <= 128 VGPRs).
constexpr int pre_threads(int n) { return (n >= 8 ? 8 : 4) * 64; }

template <int N, int MODE>
struct PreShape {
  static constexpr int FD = MODE == kFull ? 2 * N + N * N : (MODE == kNoHres ? 2 * N : N);
  static constexpr int NT = (FD + 15) / 16;  // 16-wide MFMA column tiles
  static constexpr int FDP = NT * 16;
  static constexpr int WAVES = pre_threads(N) / 64;
};

template <int N, int MODE, int KB>
__global__ __launch_bounds__(pre_threads(N)) void pre_mfma_kernel(PreArgs a) {
  using S = PreShape<N, MODE>;
  constexpr int FD = S::FD;
  constexpr int NT = S::NT;
  constexpr int FDP = S::FDP;
  constexpr int WAVES = S::WAVES;
  constexpr int T = WAVES * 64;
  constexpr int TM = kTokTile;
  constexpr int G = N * N;

  __shared__ float s_acc[WAVES][TM][FDP];
  __shared__ float s_ss[WAVES][TM];
  __shared__ float s_mix[TM * FD];
  __shared__ float s_hpre[TM][N];
  __shared__ float s_hres[MODE == kFull ? TM * G : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int r = lane & 15;   // token row inside the tile (MFMA M index)
  const int g = lane >> 4;   // 8-column group inside a 32-column block
  const int64_t M = a.M;
  const int C = a.C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const int64_t NC = (int64_t)N * C;
  const int64_t t0 = (int64_t)blockIdx.x * TM;
  const int64_t tok = t0 + r;
  const bool tok_ok = tok < M;
  const uint16_t* __restrict__ xrow = static_cast<const uint16_t*>(a.x) + (tok_ok ? tok : 0) * NC;

  // ---- 1. issue every x load of this lane up front (one HBM pass) ----------
  U32x4 xr[KB][N];
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int c = (wave + WAVES * q) * kCBlock + g * 8;
    const bool ok = tok_ok && c < C;  // C % 8 == 0: a chunk is all-in or all-out
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (ok) {
        xr[q][i] = *reinterpret_cast<const U32x4*>(xrow + (int64_t)i * C + c);
      } else {
        xr[q][i] = U32x4{{0u, 0u, 0u, 0u}};
      }
    }
  }

  // ---- 2. sum of squares + projection on MFMA --------------------------------
  f32x4_t acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;
  const bf16x8_t* __restrict__ wp = static_cast<const bf16x8_t*>(a.phi_packed);
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int cb = wave + WAVES * q;
    if (cb < NCB) {  // wave-uniform
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const U32x4 v = xr[q][i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = bf16lo(v.v[j]);
          const float hi = bf16hi(v.v[j]);
          ss = fmaf(lo, lo, ss);
          ss = fmaf(hi, hi, ss);
        }
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, v);
        const bf16x8_t* wblk = wp + (int64_t)(i * NCB + cb) * NT * 64 + lane;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bf16x8_t bv = wblk[nt * 64];
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[nt], 0, 0, 0);
        }
      }
    }
  }

  // Lanes r, r+16, r+32, r+48 hold the same token: fold their partial sums.
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);

  // ---- 3. cross-wave reduction through LDS -------------------------------------
  // MFMA 16x16 result layout: lane l holds D[4*(l/16) + j][l % 16], j = 0..3.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int j = 0; j < 4; ++j) s_acc[wave][4 * g + j][nt * 16 + r] = acc[nt][j];
  if (g == 0) s_ss[wave][r] = ss;
  __syncthreads();

  for (int idx = tid; idx < TM * FD; idx += T) {
    const int tt = idx / FD;
    const int f = idx - tt * FD;
    float sq = 0.f;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      sq += s_ss[w][tt];
      sum += s_acc[w][tt][f];
    }
    const float inv = 1.0f / sqrtf(sq / (float)NC + a.rms_eps);
    const float m = sum * inv;
    s_mix[idx] = m;
    const int64_t tk = t0 + tt;
    if (tk < M) {
      if (a.mixes_raw) a.mixes_raw[tk * FD + f] = m;
      if (a.inv_rms && f == 0) a.inv_rms[tk] = inv;
    }
  }
  __syncthreads();

  // ---- 4. gates -------------------------------------------------------------------
  {
    const int pdt = a.param_dtype;
    const float al0 = ld_any(a.alpha[0], 0, pdt);
    const float al1 = MODE == kHead ? 0.f : ld_any(a.alpha[1], 0, pdt);
    const float al2 = MODE == kFull ? ld_any(a.alpha[2], 0, pdt) : 0.f;
    for (int idx = tid; idx < TM * FD; idx += T) {
      const int tt = idx / FD;
      const int f = idx - tt * FD;
      const int64_t tk = t0 + tt;
      const bool ok = tk < M;
      const float m = s_mix[idx];
      if (f < N) {
        const float h = gate_pre(m, al0, ld_any(a.bias[0], f, pdt), a.pre_eps, kBF16);
        s_hpre[tt][f] = h;
        if (ok && a.h_pre) st_any(a.h_pre, tk * N + f, kBF16, h);
      } else if (f < 2 * N) {
        const float h = gate_post(m, al1, ld_any(a.bias[1], f - N, pdt), a.post_mult, kBF16);
        if (ok) st_any(a.h_post, tk * N + (f - N), kBF16, h);
      } else {
        const int e = f - 2 * N;
        const float h = gate_res(m, al2, ld_any(a.bias[2], e, pdt), kBF16);
        if constexpr (MODE == kFull) s_hres[tt * G + e] = h;
        if (ok && a.h_res_raw) st_any(a.h_res_raw, tk * G + e, kBF16, h);
      }
    }
  }
  __syncthreads();

  // ---- 5. Sinkhorn-Knopp, one matrix element per lane ---------------------------
  if constexpr (MODE == kFull) {
    if (a.h_res) {
      for (int e0 = 0; e0 < TM * G; e0 += T) {
        const int e = e0 + tid;
        const bool in = e < TM * G;  // groups of G lanes are all-in or all-out
        float v = in ? s_hres[e] : 0.f;
        v = sinkhorn_lane<N>(v, a.sk_iters, a.sk_eps);
        const int64_t tk = t0 + e / G;
        if (in && tk < M) st_any(a.h_res, t0 * G + e, kBF16, v);
      }
    }
  }

  // ---- 6. pre-aggregate from the held x registers ------------------------------
  uint32_t hlo[N];
  uint32_t hhi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    hlo[i] = pack_lo(s_hpre[r][i]);
    hhi[i] = pack_hi(s_hpre[r][i]);
  }
  uint16_t* __restrict__ sub = static_cast<uint16_t*>(a.sub_in);
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int c = (wave + WAVES * q) * kCBlock + g * 8;
    if (tok_ok && c < C) {
      const U32x4 pk = preagg_chunk<N>(xr[q], hlo, hhi);
      *reinterpret_cast<U32x4*>(sub + tok * C + c) = pk;
    }
  }
}

// Column blocks one wave must hold for a given C.
inline int pre_mfma_kb_needed(int n, int C) {
  const int waves = n >= 8 ? 8 : 4;
  const int ncb = (C + kCBlock - 1) / kCBlock;
  return (ncb + waves - 1) / waves;
}

template <int N, int MODE, int KB>
hipError_t launch_pre_mfma_inst(const PreArgs& a, hipStream_t s) {
  const int64_t blocks = (a.M + kTokTile - 1) / kTokTile;
  hipLaunchKernelGGL((pre_mfma_kernel<N, MODE, KB>), dim3((unsigned)blocks),
                     dim3(PreShape<N, MODE>::WAVES * 64), 0, s, a);
  return hipGetLastError();
}

// Launch the smallest instantiated KB that covers the need (KBS ascending).
template <int N, int MODE, int... KBS>
hipError_t dispatch_pre_kb(const PreArgs& a, int kb, hipStream_t s) {
  hipError_t r = hipErrorInvalidValue;
  bool done = false;
  ((!done && KBS >= kb ? (r = launch_pre_mfma_inst<N, MODE, KBS>(a, s), done = true) : false), ...);
  return r;
}

template <int N, int... KBS>
hipError_t dispatch_pre_mode(const PreArgs& a, int kb, hipStream_t s) {
  switch (a.mode) {
    case kFull: return dispatch_pre_kb<N, kFull, KBS...>(a, kb, s);
    case kNoHres: return dispatch_pre_kb<N, kNoHres, KBS...>(a, kb, s);
    case kHead:
      if constexpr (N > 1) return dispatch_pre_kb<N, kHead, KBS...>(a, kb, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

// Largest KB instantiated per n (see the mhc_pre_mfma_n*.hip files).
inline int pre_mfma_kb_max(int n) { return n >= 8 ? 4 : 8; }

// Per-n entry points, one translation unit each so they compile in parallel.
hipError_t launch_pre_mfma_n1(const PreArgs& a, int kb, hipStream_t s);
hipError_t launch_pre_mfma_n2(const PreArgs& a, int kb, hipStream_t s);
hipError_t launch_pre_mfma_n4(const PreArgs& a, int kb, hipStream_t s);
hipError_t launch_pre_mfma_n8(const PreArgs& a, int kb, hipStream_t s);

}  // namespace mhc
