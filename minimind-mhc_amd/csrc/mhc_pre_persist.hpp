// Persistent fused mHC pre phase on MFMA, bf16 streams (gfx950).
//
// Same arithmetic as pre_mfma_kernel (mhc_pre_mfma.hpp), scheduled for HBM:
//   * one 8-wave workgroup per CU walks the 16-token tiles blockIdx.x,
//     blockIdx.x + gridDim.x, ... until the tiles run out;
//   * wave w owns the 32-column blocks cb = w, w + 8, ... of every stream;
//   * phi stays resident for the workgroup's lifetime, as MFMA B operands: the
//     first NREG 16-column tiles in registers, the next NLDS tiles in LDS (the
//     last, partial tile stored compactly: lanes past its real columns read a
//     shared zero block), any rest re-read from L2 per tile;
//   * x tiles are DEPTH-buffered in registers: DEPTH - 1 tiles are in flight
//     while one runs its MFMAs, cross-wave reduction, gates, Sinkhorn and
//     pre-aggregate.  Loaded HBM latency on MI355X is several microseconds,
//     so one tile (96 KiB per CU at n=4, C=768) in flight cannot keep HBM
//     busy; DEPTH = 3 keeps two.
//   * x loads and sub_in stores are raw buffer ops bounded by a per-tile
//     descriptor: missing tokens / columns are zero-filled (or dropped) by
//     hardware, so no load sits behind a branch and the compiler waits only
//     for the tile it is about to use;
//   * the tile loop issues no other global load: the vector-memory counter
//     retires in order, so waiting on any load issued after a prefetch would
//     also wait for the prefetch.  Gate scalars and biases are read once, before
//     the first x load, and kept in LDS as fp32.
// Per tile: two workgroup barriers (partials written; gates written).
//
// Reference semantics: model/mhc_fused.py:163-268, :533-559, :47-56,
// :820-830; model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195.
#pragma once

#include "mhc_pre_mfma.hpp"

namespace mhc {

constexpr int kPersistWaves = 8;
constexpr int kLdsBytes = 163840;  // LDS per CU on gfx950

// Gate parameters in LDS: alpha_pre, alpha_post, alpha_res, then bias_pre[n],
// bias_post[n], bias_res[n*n] (fp32).
template <int N>
struct GateParams {
  static constexpr int kCount = 3 + 2 * N + N * N;
  static constexpr int kBiasPre = 3;
  static constexpr int kBiasPost = 3 + N;
  static constexpr int kBiasRes = 3 + 2 * N;
};

template <int N, int FD>
struct PersistShared {
  float prm[GateParams<N>::kCount];
  float acc[kPersistWaves][kTokTile][FD];  // per-wave partial projections
  float ss[kPersistWaves][kTokTile];       // per-wave partial sums of squares
  float hpre[kTokTile][N];
  float hres[kTokTile * N * N];
  U32x4 zero;                              // B operand of padding columns
};

template <int N, int MODE, int KB>
struct PersistPlan {
  using S = PreShape<N, MODE>;
  static constexpr int FD = S::FD;
  static constexpr int NT = S::NT;
  static constexpr int G = N * N;
  static constexpr int LAST_COLS = FD - 16 * (NT - 1);  // real columns of the last tile
  // registers: x buffers first, then whole phi tiles
  static constexpr int kRegBudget = 160;
  static constexpr int XTILE = KB * N * 4;  // VGPRs of one x tile (and of one phi tile)
  static constexpr int DEPTH = 3 * XTILE <= kRegBudget ? 3 : 2;
  static constexpr int REG_LEFT = kRegBudget - DEPTH * XTILE;
  static constexpr int REG_FIT = REG_LEFT > 0 ? REG_LEFT / XTILE : 0;
  static constexpr int NREG = REG_FIT < NT ? REG_FIT : NT;
  // LDS: shared scratch, then phi tiles NREG.. while they fit
  static constexpr int SHARED = (int)sizeof(PersistShared<N, FD>);
  static constexpr int cols(int t) { return t == NT - 1 ? LAST_COLS : 16; }
  static constexpr int tile_lds(int t) { return kPersistWaves * KB * N * 4 * cols(t) * 16; }
  static constexpr int lds_tiles() {
    int used = SHARED + 256;
    int k = 0;
    for (int t = NREG; t < NT; ++t) {
      if (used + tile_lds(t) > kLdsBytes) break;
      used += tile_lds(t);
      ++k;
    }
    return k;
  }
  static constexpr int NLDS = lds_tiles();
  static constexpr int lds_base(int t) {  // byte offset of phi tile t inside lds_w
    int off = 0;
    for (int u = NREG; u < t; ++u) off += tile_lds(u);
    return off;
  }
  static constexpr int LDS_W = lds_base(NREG + NLDS) > 0 ? lds_base(NREG + NLDS) : 16;
  static constexpr int WR = NREG > 0 ? NREG : 1;  // register array extent (>= 1)
};

// Tokens of a tile that exist (0 for a tile past the end).
__device__ __forceinline__ int tile_tokens(int64_t tile, int64_t ntiles, int64_t M) {
  if (tile >= ntiles) return 0;
  const int64_t left = M - tile * kTokTile;
  return left < kTokTile ? (int)left : kTokTile;
}

// Load this lane's x chunks of one tile.  The descriptor covers the tile's
// existing tokens (valid * n*C * 2 bytes); a lane whose token is missing has a
// lane offset past that bound and a column past C gets kBufOob, so either
// reads zeros.  The per-(stream, block) part of the offset is wave-uniform
// and travels in the scalar offset.
template <int N, int KB>
__device__ __forceinline__ void persist_load_tile(U32x4 (&xr)[KB][N], const uint16_t* __restrict__ x,
                                                  int64_t tile, int64_t ntiles, int64_t M, int C,
                                                  int wave, int r, int g) {
  const int NC = N * C;
  const int valid = tile_tokens(tile, ntiles, M);
  const auto rsrc = make_rsrc(x + (valid > 0 ? tile * kTokTile * (int64_t)NC : 0),
                              (uint32_t)valid * (uint32_t)NC * 2u);
  const uint32_t lane_off = (uint32_t)(r * NC + g * 8) * 2u;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int c0 = (wave + kPersistWaves * q) * kCBlock;
    const uint32_t voff = c0 + g * 8 < C ? lane_off : kBufOob;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int soff = (i * C + c0) * 2;
      xr[q][i] = __builtin_bit_cast(U32x4,
                                    __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)voff, soff, 0));
    }
  }
}

template <int N, int MODE, int KB>
__device__ __forceinline__ void persist_tile(
    const PreArgs& a, PersistShared<N, PersistPlan<N, MODE, KB>::FD>& sh, const U32x4 (&xr)[KB][N],
    const bf16x8_t (&wreg)[KB][N][PersistPlan<N, MODE, KB>::WR], const unsigned char* lds_w,
    int64_t tile, int tid, int lane, int wave) {
  using P = PersistPlan<N, MODE, KB>;
  using GP = GateParams<N>;
  constexpr int FD = P::FD;
  constexpr int NT = P::NT;
  constexpr int G = P::G;
  constexpr int T = kPersistWaves * 64;
  constexpr int TM = kTokTile;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t M = a.M;
  const int C = a.C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const int64_t NC = (int64_t)N * C;
  const int64_t t0 = tile * TM;

  // ---- sum of squares (bf16 dot2) + projection (MFMA) ----------------------
  f32x4_t acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;
  const bf16x8_t* __restrict__ wp = static_cast<const bf16x8_t*>(a.phi_packed);
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int cb = wave + kPersistWaves * q;
    if (cb < NCB) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const U32x4 v = xr[q][i];
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = dot2_bf16(v.v[j], v.v[j], ss);
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, v);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          bf16x8_t bv;
          if (nt < P::NREG) {  // compile-time after unrolling
            bv = wreg[q][i][nt < P::NREG ? nt : 0];
          } else if (nt < P::NREG + P::NLDS) {
            const int cols = P::cols(nt);
            const unsigned char* src =
                r < cols ? lds_w + P::lds_base(nt) +
                               ((((wave * KB + q) * N + i) * 4 + g) * cols + r) * 16
                         : reinterpret_cast<const unsigned char*>(&sh.zero);
            bv = *reinterpret_cast<const bf16x8_t*>(src);
          } else {
            bv = wp[((int64_t)(i * NCB + cb) * NT + nt) * 64 + lane];
          }
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[nt], 0, 0, 0);
        }
      }
    }
  }
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  // MFMA 16x16 result layout: lane l holds D[4*(l/16) + j][l % 16], j = 0..3.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    if (nt * 16 + r < FD)
#pragma unroll
      for (int j = 0; j < 4; ++j) sh.acc[wave][4 * g + j][nt * 16 + r] = acc[nt][j];
  if (g == 0) sh.ss[wave][r] = ss;
  __syncthreads();

  // ---- reduce partials, inv_rms, gates -----------------------------------------
  for (int idx = tid; idx < TM * FD; idx += T) {
    const int tt = idx / FD;
    const int f = idx - tt * FD;
    float sq = 0.f;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kPersistWaves; ++w) {
      sq += sh.ss[w][tt];
      sum += sh.acc[w][tt][f];
    }
    const float inv = 1.0f / sqrtf(sq / (float)NC + a.rms_eps);
    const float m = sum * inv;
    const int64_t tk = t0 + tt;
    const bool ok = tk < M;
    if (ok) {
      if (a.mixes_raw) a.mixes_raw[tk * FD + f] = m;
      if (a.inv_rms && f == 0) a.inv_rms[tk] = inv;
    }
    if (f < N) {
      const float h = gate_pre(m, sh.prm[0], sh.prm[GP::kBiasPre + f], a.pre_eps, kBF16);
      sh.hpre[tt][f] = h;
      if (ok && a.h_pre) st_any(a.h_pre, tk * N + f, kBF16, h);
    } else if (f < 2 * N) {
      const float h = gate_post(m, sh.prm[1], sh.prm[GP::kBiasPost + f - N], a.post_mult, kBF16);
      if (ok) st_any(a.h_post, tk * N + (f - N), kBF16, h);
    } else {
      const int e = f - 2 * N;
      const float h = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e], kBF16);
      if constexpr (MODE == kFull) sh.hres[tt * G + e] = h;
      if (ok && a.h_res_raw) st_any(a.h_res_raw, tk * G + e, kBF16, h);
    }
  }
  __syncthreads();

  // ---- Sinkhorn-Knopp, one matrix element per lane -----------------------------
  if constexpr (MODE == kFull) {
    if (a.h_res && wave * 64 < TM * G) {  // wave-uniform: whole groups only
      const int e = tid;
      float v = e < TM * G ? sh.hres[e] : 0.f;
      v = sinkhorn_lane<N>(v, a.sk_iters, a.sk_eps);
      if (e < TM * G && t0 + e / G < M) st_any(a.h_res, t0 * G + e, kBF16, v);
    }
  }

  // ---- pre-aggregate from the held x registers ---------------------------------
  uint32_t hlo[N];
  uint32_t hhi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    hlo[i] = pack_lo(sh.hpre[r][i]);
    hhi[i] = pack_hi(sh.hpre[r][i]);
  }
  const int valid = (int)(M - t0 < TM ? M - t0 : TM);
  const auto rsub = make_rsrc(static_cast<uint16_t*>(a.sub_in) + t0 * C, (uint32_t)valid * C * 2u);
  const uint32_t lane_off = (uint32_t)(r * C + g * 8) * 2u;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int c0 = (wave + kPersistWaves * q) * kCBlock;
    const U32x4 pk = preagg_chunk<N>(xr[q], hlo, hhi);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, pk), rsub,
                                           (int)(c0 + g * 8 < C ? lane_off : kBufOob), c0 * 2, 0);
  }
}

template <int N, int MODE, int KB>
__global__ __launch_bounds__(kPersistWaves * 64) void pre_persist_kernel(PreArgs a, int64_t ntiles) {
  using P = PersistPlan<N, MODE, KB>;
  static_assert(P::SHARED + 256 + (P::NLDS > 0 ? P::LDS_W : 0) <= kLdsBytes, "LDS budget");
  __shared__ PersistShared<N, P::FD> sh;
  __shared__ __attribute__((aligned(16))) unsigned char lds_w[P::LDS_W];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int C = a.C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(a.x);
  const int64_t step = gridDim.x;

  // Gate parameters first, so the waits for them never cover a streaming load.
  using GP = GateParams<N>;
  float prm = 0.f;
  if (tid < GP::kCount) {
    const int pdt = a.param_dtype;
    if (tid < 3) {
      const bool used = tid == 0 || (tid == 1 && MODE != kHead) || (tid == 2 && MODE == kFull);
      if (used) prm = ld_any(a.alpha[tid], 0, pdt);
    } else if (tid < GP::kBiasPost) {
      prm = ld_any(a.bias[0], tid - GP::kBiasPre, pdt);
    } else if (tid < GP::kBiasRes) {
      if (MODE != kHead) prm = ld_any(a.bias[1], tid - GP::kBiasPost, pdt);
    } else {
      if (MODE == kFull) prm = ld_any(a.bias[2], tid - GP::kBiasRes, pdt);
    }
  }

  // phi, resident for the workgroup's lifetime (unconditional buffer loads:
  // column blocks past C read zeros).  Issued before the x loads so that
  // waiting for it (to fill LDS) does not wait for x.
  if (tid == 0) sh.zero = U32x4{{0u, 0u, 0u, 0u}};
  bf16x8_t wreg[KB][N][P::WR];
  {
    const uint32_t wbytes = (uint32_t)(N * NCB * P::NT) * 64u * 16u;
    const auto wr = make_rsrc(a.phi_packed, wbytes);
#pragma unroll
    for (int nt = 0; nt < P::NREG + P::NLDS; ++nt) {
#pragma unroll
      for (int q = 0; q < KB; ++q) {
        const int cb = wave + kPersistWaves * q;
#pragma unroll
        for (int i = 0; i < N; ++i) {
          const uint32_t off = cb < NCB
              ? (uint32_t)(((i * NCB + cb) * P::NT + nt) * 64 + lane) * 16u : kBufOob;
          const U32x4 w = buf_load16(wr, off);
          if (nt < P::NREG) {
            wreg[q][i][nt < P::NREG ? nt : 0] = __builtin_bit_cast(bf16x8_t, w);
          } else {
            const int cols = P::cols(nt);
            if (r < cols)
              *reinterpret_cast<U32x4*>(lds_w + P::lds_base(nt) +
                                        ((((wave * KB + q) * N + i) * 4 + g) * cols + r) * 16) = w;
          }
        }
      }
    }
  }
  if (tid < GP::kCount) sh.prm[tid] = prm;

  U32x4 xa[KB][N];
  U32x4 xb[KB][N];
  U32x4 xc[P::DEPTH == 3 ? KB : 1][N];
  int64_t tile = blockIdx.x;
  persist_load_tile<N, KB>(xa, x, tile, ntiles, a.M, C, wave, r, g);
  persist_load_tile<N, KB>(xb, x, tile + step, ntiles, a.M, C, wave, r, g);
  __syncthreads();  // gate parameters, zero block and phi tiles visible

  if constexpr (P::DEPTH == 3) {
    while (tile < ntiles) {  // uniform across the workgroup
      persist_load_tile<N, KB>(xc, x, tile + 2 * step, ntiles, a.M, C, wave, r, g);
      persist_tile<N, MODE, KB>(a, sh, xa, wreg, lds_w, tile, tid, lane, wave);
      if (tile + step >= ntiles) break;
      persist_load_tile<N, KB>(xa, x, tile + 3 * step, ntiles, a.M, C, wave, r, g);
      persist_tile<N, MODE, KB>(a, sh, xb, wreg, lds_w, tile + step, tid, lane, wave);
      if (tile + 2 * step >= ntiles) break;
      persist_load_tile<N, KB>(xb, x, tile + 4 * step, ntiles, a.M, C, wave, r, g);
      persist_tile<N, MODE, KB>(a, sh, xc, wreg, lds_w, tile + 2 * step, tid, lane, wave);
      tile += 3 * step;
    }
  } else {
    while (tile < ntiles) {
      persist_tile<N, MODE, KB>(a, sh, xa, wreg, lds_w, tile, tid, lane, wave);
      if (tile + step >= ntiles) break;
      persist_load_tile<N, KB>(xa, x, tile + 2 * step, ntiles, a.M, C, wave, r, g);
      persist_tile<N, MODE, KB>(a, sh, xb, wreg, lds_w, tile + step, tid, lane, wave);
      if (tile + 2 * step >= ntiles) break;
      persist_load_tile<N, KB>(xb, x, tile + 3 * step, ntiles, a.M, C, wave, r, g);
      tile += 2 * step;
    }
  }
}

// Column blocks per wave for the persistent kernel.
inline int persist_kb_needed(int C) {
  const int ncb = (C + kCBlock - 1) / kCBlock;
  return (ncb + kPersistWaves - 1) / kPersistWaves;
}

// Launch with one workgroup per CU (fewer when there are fewer tiles).
template <int N, int MODE, int KB>
hipError_t launch_pre_persist_inst(const PreArgs& a, int num_cus, hipStream_t s) {
  const int64_t ntiles = (a.M + kTokTile - 1) / kTokTile;
  const int64_t grid = ntiles < num_cus ? ntiles : num_cus;
  hipLaunchKernelGGL((pre_persist_kernel<N, MODE, KB>), dim3((unsigned)grid),
                     dim3(kPersistWaves * 64), 0, s, a, ntiles);
  return hipGetLastError();
}

template <int N, int MODE, int... KBS>
hipError_t dispatch_persist_kb(const PreArgs& a, int kb, int num_cus, hipStream_t s) {
  hipError_t r = hipErrorInvalidValue;
  bool done = false;
  ((!done && KBS >= kb ? (r = launch_pre_persist_inst<N, MODE, KBS>(a, num_cus, s), done = true)
                       : false),
   ...);
  return r;
}

template <int N>
hipError_t dispatch_persist_mode(const PreArgs& a, int kb, int num_cus, hipStream_t s) {
  switch (a.mode) {
    case kFull: return dispatch_persist_kb<N, kFull, 1, 2, 3, 4>(a, kb, num_cus, s);
    case kNoHres: return dispatch_persist_kb<N, kNoHres, 1, 2, 3, 4>(a, kb, num_cus, s);
    case kHead:
      if constexpr (N > 1) return dispatch_persist_kb<N, kHead, 1, 2, 3, 4>(a, kb, num_cus, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

// Per-n entry points (mhc_pre_persist_n*.hip).
hipError_t launch_pre_persist_n1(const PreArgs& a, int kb, int num_cus, hipStream_t s);
hipError_t launch_pre_persist_n2(const PreArgs& a, int kb, int num_cus, hipStream_t s);
hipError_t launch_pre_persist_n4(const PreArgs& a, int kb, int num_cus, hipStream_t s);

}  // namespace mhc
