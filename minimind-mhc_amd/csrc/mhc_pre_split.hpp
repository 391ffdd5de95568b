// Persistent fused mHC pre phase for fp32 streams and fp32 phi (the layout of
// the reference's trainers: an fp32 model under bf16 autocast,
// trainer/train_pretrain.py:129-130, keeps the mHC stream in fp32,
// model/mhc_fused.py:733).  bf16 MFMA on split operands:
//
//   x   = x_hi + x_lo,     x_hi = bf16(x),   x_lo = bf16(x - x_hi)
//   phi = p_hi + p_lo      (the same split)
//   x . phi ~= (x_hi + x_lo) . (p_hi + p_lo)        (all four products, each
//                                                    exact in fp32)
// The split keeps 16 of fp32's 24 significant bits of each operand: measured
// max-norm relative error of the projection 3.3e-6 at n*C = 3072 against a
// float64 product (the fp32 bar is 1e-5).  One MFMA forms all four products:
//   * A rows 0..7 hold x_hi of the tile's 8 tokens, rows 8..15 x_lo of the same
//     tokens.  Lane (g, r) loads the 4 fp32 of token r & 7 at columns
//     8g + 4 (r >> 3) .. + 3 of the 32-column block (a tile row of one block is
//     one 128-byte line), forms both splits of them, and swaps the half its
//     partner lane r ^ 8 needs by DPP (row_ror:8);
//   * the packed phi image has 16-column B tiles of 8 features each: columns
//     0..7 p_hi, columns 8..15 p_lo of the same features;
//   * so D[t][c] + D[t+8][c] + D[t][c+8] + D[t+8][c+8] is token t's projection
//     onto feature 8u + c (two butterflies: lane ^ 32, then lane ^ 8).
// Everything else is fp32: the sum of squares, inv_rms, the gates (no
// rounding points in an fp32 stream), the Sinkhorn and the pre-aggregate
// (each product rounded, then summed over streams in order).
//
// Schedule: as pre_persist_kernel (one 8-wave workgroup per CU walking 8-token
// tiles; x double-buffered in registers; one barrier a tile; the Sinkhorn of
// the previous tile on the first waves).  The next tile's loads go out in
// three batches: at the step's start, after the partials (before the
// barrier), and after the pre-aggregate, so the last batch follows the
// step's scattered gate stores instead of preceding them.  Measured at C2
// (16384 tokens, n = 4, C = 768, with the saved outputs of a training
// forward): 54.4 -> 52.4 us against the second batch after the barrier; the
// last batch ahead of the gate stores measured 60 us, all loads at the
// step's start 63 us.  An 8-token fp32 tile is 96 KiB, the size of the bf16 kernel's
// 16-token tile, and takes the same registers.  phi: the first NREG B tiles
// in registers, the next NLDS in LDS, any rest read from L2.
//
// Reference semantics: model/mhc_fused.py:163-268 (fused kernel), :533-559,
// :47-56; model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195.
#pragma once

#include "mhc_pre_persist.hpp"

namespace mhc {

constexpr int kSplitTok = 8;  // tokens per tile

template <int N, int MODE, int KB>
struct SplitPlan {
  using S = PreShape<N, MODE>;
  static constexpr int FD = S::FD;
  static constexpr int NU = (FD + 7) / 8;  // B tiles: 8 features, hi | lo columns
  static constexpr int NN = N * N;
  static constexpr int NB = N * KB;        // 32-column blocks per wave
  static constexpr int XT = NB * 4;        // VGPRs of one x tile, and of one phi tile
  // Registers: two x tiles, then whole phi tiles while they fit in 192 (176
  // for the 64-VGPR tiles of C = 1024, whose working set is larger).
  static constexpr int REG_FIT = ((XT > 48 ? 176 : 192) - 2 * XT) / XT;
  static constexpr int NREG = REG_FIT < NU ? (REG_FIT > 0 ? REG_FIT : 0) : NU;
  static constexpr int WR = NREG > 0 ? NREG : 1;
  static constexpr int TILE_LDS = kPersistWaves * NB * 1024;  // bytes of one phi tile in LDS
  static constexpr int SHARED_EST = 24 * 1024;                // partials and the rest, rounded up
  static constexpr int LDS_FIT = (kLdsBytes - SHARED_EST) / TILE_LDS;
  static constexpr int NLDS = NU - NREG < LDS_FIT ? NU - NREG : LDS_FIT;
  static constexpr int LDS_W = NLDS > 0 ? NLDS * TILE_LDS : 16;
  // Column blocks of the next tile loaded at the three points of a step:
  // [0, B1) at its start, [B1, B2) after the partials, [B2, KB) at its end.
  static constexpr int B1 = (KB + 2) / 3;
  static constexpr int B2 = (2 * KB + 2) / 3;
  // Waves that run the Sinkhorn of the previous tile (one element per lane).
  static constexpr int SK_WAVES = MODE == kFull ? (kSplitTok * NN + 63) / 64 : 0;
  static constexpr int GATE_LANES = (kPersistWaves - SK_WAVES) * 64;
  static constexpr int POST_WAVE = kPersistWaves - 1;
  static_assert(SK_WAVES < kPersistWaves, "gates need at least one wave");
  static_assert(kSplitTok * N <= 64, "one wave holds a tile's h_pre");
};

template <int N, int MODE, int KB>
struct SplitShared {
  using P = SplitPlan<N, MODE, KB>;
  float prm[GateParams<N>::kCount];
  float acc[2][kPersistWaves][kSplitTok][P::FD];  // per-wave partial projections, 2 slots
  float ss[2][kPersistWaves][kSplitTok];          // per-wave partial sums of squares
  float hres[2][kSplitTok * (MODE == kFull ? P::NN : 1)];
};

// Buffer descriptor over one tile's fp32 x (or sub_in) rows; no records past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t split_rsrc(const void* base, int64_t tile,
                                                             int64_t M, int row_floats) {
  const int64_t t0 = tile * kSplitTok;
  const int valid = t0 >= M ? 0 : (M - t0 < kSplitTok ? (int)(M - t0) : kSplitTok);
  return make_rsrc(static_cast<const float*>(base) + (valid > 0 ? t0 * row_floats : 0),
                   (uint32_t)valid * (uint32_t)row_floats * 4u);
}

// Column part of lane (g, r)'s offset in column block q of this wave (floats);
// -1 past C.
__device__ __forceinline__ int split_col(int q, int wave, int g, int r, int C) {
  const int c0 = (wave + kPersistWaves * q) * kCBlock;
  return c0 + 8 * g < C ? c0 + 8 * g + 4 * (r >> 3) : -1;
}

// Load column blocks [Q0, Q1) of this lane's x chunks of one tile.
template <int N, int KB, int Q0, int Q1>
__device__ __forceinline__ void split_load(U32x4 (&xr)[KB][N], __amdgpu_buffer_rsrc_t rsrc, int C,
                                           int wave, int lane) {
  const int r = lane & 15;
  const int g = lane >> 4;
  const uint32_t row = (uint32_t)((r & 7) * N * C) * 4u;
#pragma unroll
  for (int q = Q0; q < Q1; ++q) {
    const int col = split_col(q, wave, g, r, C);
#pragma unroll
    for (int i = 0; i < N; ++i)
      xr[q][i] = buf_load16_nt<kNtSc1>(rsrc, col < 0 ? kBufOob : row + (uint32_t)(i * C + col) * 4u, 0);
  }
}

// A operand of one block from this lane's 4 fp32: rows 0..7 take x_hi, rows
// 8..15 x_lo, of k = 8g .. 8g + 7 (the first half owned by lane r, the second
// by lane r + 8).
__device__ __forceinline__ bf16x8_t split_operand(const U32x4& v, bool hi_lane) {
  const float x0 = __uint_as_float(v.v[0]), x1 = __uint_as_float(v.v[1]);
  const float x2 = __uint_as_float(v.v[2]), x3 = __uint_as_float(v.v[3]);
  const uint32_t h01 = pack_bf16x2(x0, x1);
  const uint32_t h23 = pack_bf16x2(x2, x3);
  const uint32_t l01 = pack_bf16x2(x0 - bf16lo(h01), x1 - bf16hi(h01));
  const uint32_t l23 = pack_bf16x2(x2 - bf16lo(h23), x3 - bf16hi(h23));
  // A hi lane's partner (a lo lane) needs this lane's lo half, and the reverse.
  const uint32_t s01 = hi_lane ? l01 : h01;
  const uint32_t s23 = hi_lane ? l23 : h23;
  const uint32_t p01 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s01, kDppRor8, 0xF, 0xF, true);
  const uint32_t p23 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s23, kDppRor8, 0xF, 0xF, true);
  U32x4 a;
  a.v[0] = hi_lane ? h01 : p01;
  a.v[1] = hi_lane ? h23 : p23;
  a.v[2] = hi_lane ? p01 : l01;
  a.v[3] = hi_lane ? p23 : l23;
  return __builtin_bit_cast(bf16x8_t, a);
}

// ---- phase 1: sum of squares + MFMA partial projections -> LDS -----------
template <int N, int MODE, int KB>
__device__ __forceinline__ void split_partials(const PreArgs& a, SplitShared<N, MODE, KB>& sh,
                                               const U32x4 (&xr)[KB][N],
                                               const bf16x8_t (&wreg)[KB][N][SplitPlan<N, MODE, KB>::WR],
                                               const unsigned char* lds_w, int slot, int lane, int wave) {
  using P = SplitPlan<N, MODE, KB>;
  constexpr int FD = P::FD;
  constexpr int NU = P::NU;
  const int r = lane & 15;
  const int g = lane >> 4;
  const bool hi_lane = r < 8;
  const int NCB = (a.C + kCBlock - 1) / kCBlock;
  const auto wr = make_rsrc(a.phi_packed, (uint32_t)(N * NCB * NU) * 1024u);
  f32x4_t acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int cb = wave + kPersistWaves * q;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const U32x4 v = xr[q][i];
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = fmaf(__uint_as_float(v.v[j]), __uint_as_float(v.v[j]), ss);
      const bf16x8_t av = split_operand(v, hi_lane);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        bf16x8_t bv;
        if (u < P::NREG) {  // compile-time after unrolling
          bv = wreg[q][i][u < P::NREG ? u : 0];
        } else if (u < P::NREG + P::NLDS) {
          bv = *reinterpret_cast<const bf16x8_t*>(
              lds_w + (u - P::NREG) * P::TILE_LDS + (((wave * KB + q) * N + i) * 64 + lane) * 16);
        } else {
          const uint32_t off =
              cb < NCB ? (uint32_t)(((i * NCB + cb) * NU + u) * 64 + lane) * 16u : kBufOob;
          bv = __builtin_bit_cast(bf16x8_t, buf_load16(wr, off));
        }
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[u], 0, 0, 0);
      }
    }
  }
  // Token r & 7's squares live in lanes r, r ^ 8 of every lane group.
  ss = ss + dpp_f<kDppRor8>(ss);
  ss = ss + xor_lane16(ss);
  ss = ss + xor_lane32(ss);
  if (lane < kSplitTok) sh.ss[slot][wave][lane] = ss;
  // Lane (g, c) holds D[4g + j][c]: fold rows t + 8 (lane ^ 32) and columns
  // c + 8 (lane ^ 8) into lanes g < 2, c < 8: token 4g + j, feature 8u + c.
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = acc[u][j];
      v = v + xor_lane32(v);
      v = v + dpp_f<kDppRor8>(v);
      if (g < 2 && r < 8 && 8 * u + r < FD) sh.acc[slot][wave][4 * g + j][8 * u + r] = v;
    }
}

template <int N, int MODE, int KB>
__device__ __forceinline__ float split_inv_rms(const SplitShared<N, MODE, KB>& sh, int slot, int tt,
                                               float nc, float eps) {
  float sq = 0.f;
#pragma unroll
  for (int w = 0; w < kPersistWaves; ++w) sq += sh.ss[slot][w][tt];
  return 1.0f / sqrtf(sq / nc + eps);
}

template <int N, int MODE, int KB>
__device__ __forceinline__ float split_mix(const SplitShared<N, MODE, KB>& sh, int slot, int tt, int f,
                                           float inv) {
  float sum = 0.f;
#pragma unroll
  for (int w = 0; w < kPersistWaves; ++w) sum += sh.acc[slot][w][tt][f];
  return sum * inv;
}

// h_pre of (token lane / N, stream lane % N) for every wave (0 past the tile);
// wave POST_WAVE writes h_pre, inv_rms, h_post and the pre / post mixes.
template <int N, int MODE, int KB>
__device__ __forceinline__ float split_pre_post(const PreArgs& a, const SplitShared<N, MODE, KB>& sh,
                                                int64_t tile, int slot, int lane, int wave) {
  using P = SplitPlan<N, MODE, KB>;
  using GP = GateParams<N>;
  constexpr int FD = P::FD;
  float hp = 0.f;
  if (lane < kSplitTok * N) {
    const int tt = lane / N;
    const int i = lane % N;
    const float inv = split_inv_rms(sh, slot, tt, (float)(N * a.C), a.rms_eps);
    const float m = split_mix(sh, slot, tt, i, inv);
    hp = gate_pre(m, sh.prm[0], sh.prm[GP::kBiasPre + i], a.pre_eps, kF32);
    if (wave == P::POST_WAVE) {
      const int64_t tk = tile * kSplitTok + tt;
      if (tk < a.M) {
        if (a.h_pre) static_cast<float*>(a.h_pre)[tk * N + i] = hp;
        if (a.inv_rms && i == 0) a.inv_rms[tk] = inv;
        if (a.mixes_raw) a.mixes_raw[tk * FD + i] = m;
        if constexpr (MODE != kHead) {
          const float mp = split_mix(sh, slot, tt, N + i, inv);
          static_cast<float*>(a.h_post)[tk * N + i] =
              gate_post(mp, sh.prm[1], sh.prm[GP::kBiasPost + i], a.post_mult, kF32);
          if (a.mixes_raw) a.mixes_raw[tk * FD + N + i] = mp;
        }
      }
    }
  }
  return hp;
}

// h_res logits of the tile, one (token, element) per gate lane, into LDS slot
// `slot` for the next step's Sinkhorn.
template <int N, int MODE, int KB>
__device__ __forceinline__ void split_res_gates(const PreArgs& a, SplitShared<N, MODE, KB>& sh,
                                                int64_t tile, int slot, int idx0) {
  using P = SplitPlan<N, MODE, KB>;
  using GP = GateParams<N>;
  constexpr int FD = P::FD;
  constexpr int NN = P::NN;
  for (int idx = idx0; idx < kSplitTok * NN; idx += P::GATE_LANES) {
    const int tt = idx / NN;
    const int e = idx % NN;
    const float inv = split_inv_rms(sh, slot, tt, (float)(N * a.C), a.rms_eps);
    const float m = split_mix(sh, slot, tt, 2 * N + e, inv);
    const float h = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e], kF32);
    sh.hres[slot][idx] = h;
    const int64_t tk = tile * kSplitTok + tt;
    if (tk < a.M) {
      if (a.h_res_raw) static_cast<float*>(a.h_res_raw)[tk * NN + e] = h;
      if (a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e] = m;
    }
  }
}

// Sinkhorn-Knopp of tile `tile` from an LDS slot, one element per lane of the
// first SK_WAVES waves.
template <int N>
__device__ __forceinline__ void split_sinkhorn(const PreArgs& a, const float* hres, int64_t tile,
                                               int tid) {
  constexpr int NN = N * N;
  const int64_t t0 = tile * kSplitTok;
  const int e = tid;
  float v = e < kSplitTok * NN ? hres[e] : 0.f;
  v = sinkhorn_lane<N>(v, a.sk_iters, a.sk_eps);
  if (e < kSplitTok * NN && t0 + e / NN < a.M) static_cast<float*>(a.h_res)[t0 * NN + e] = v;
}

// Pre-aggregate from the held x registers: lane (g, r) forms token r & 7's 4
// columns of each of its blocks, sum_i h_i * x_i in fp32 (each product
// rounded, then added in stream order).
template <int N, int KB>
__device__ __forceinline__ void split_preagg(const PreArgs& a, const U32x4 (&xr)[KB][N],
                                             const float (&h)[N], int64_t tile, int lane, int wave) {
  const int r = lane & 15;
  const int g = lane >> 4;
  const int C = a.C;
  const auto rs = split_rsrc(a.sub_in, tile, a.M, C);
  const uint32_t row = (uint32_t)((r & 7) * C) * 4u;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int col = split_col(q, wave, g, r, C);
    U32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = mul_nc(h[0], __uint_as_float(xr[q][0].v[j]));
#pragma unroll
      for (int i = 1; i < N; ++i) s = __fadd_rn(s, mul_nc(h[i], __uint_as_float(xr[q][i].v[j])));
      o.v[j] = __float_as_uint(s);
    }
    // The whole offset in the vector offset, the scalar offset the literal 0:
    // a 128-bit store reads its data registers after issue (see persist_preagg).
    buf_store16_nt<kNt>(rs, col < 0 ? kBufOob : row + (uint32_t)col * 4u, o);
  }
}

template <int N, int MODE, int KB>
__device__ __forceinline__ void split_step(const PreArgs& a, SplitShared<N, MODE, KB>& sh,
                                           const U32x4 (&xr)[KB][N], U32x4 (&xn)[KB][N],
                                           const bf16x8_t (&wreg)[KB][N][SplitPlan<N, MODE, KB>::WR],
                                           const unsigned char* lds_w, int64_t tile, int64_t prev,
                                           int slot, int tid, int lane, int wave) {
  using P = SplitPlan<N, MODE, KB>;
  const int r = lane & 15;
  const auto rn = split_rsrc(a.x, tile + gridDim.x, a.M, N * a.C);
  split_load<N, KB, 0, P::B1>(xn, rn, a.C, wave, lane);
  split_partials<N, MODE, KB>(a, sh, xr, wreg, lds_w, slot, lane, wave);
  split_load<N, KB, P::B1, P::B2>(xn, rn, a.C, wave, lane);
  __syncthreads();
  if constexpr (MODE == kFull) {
    if (wave < P::SK_WAVES && prev >= 0 && a.h_res) split_sinkhorn<N>(a, sh.hres[slot ^ 1], prev, tid);
  }
  const float hp = split_pre_post<N, MODE, KB>(a, sh, tile, slot, lane, wave);
  if constexpr (MODE == kFull) {
    if (wave >= P::SK_WAVES) split_res_gates<N, MODE, KB>(a, sh, tile, slot, tid - P::SK_WAVES * 64);
  }
  float h[N];
#pragma unroll
  for (int i = 0; i < N; ++i) h[i] = __shfl(hp, (r & 7) * N + i, 64);
  split_preagg<N, KB>(a, xr, h, tile, lane, wave);
  split_load<N, KB, P::B2, KB>(xn, rn, a.C, wave, lane);
}

template <int N, int MODE, int KB>
__global__ __launch_bounds__(kPersistWaves * 64) void pre_split_kernel(PreArgs a, int64_t ntiles) {
  using P = SplitPlan<N, MODE, KB>;
  static_assert(sizeof(SplitShared<N, MODE, KB>) <= P::SHARED_EST, "partials estimate");
  static_assert(sizeof(SplitShared<N, MODE, KB>) + P::LDS_W <= kLdsBytes, "LDS budget");
  __shared__ SplitShared<N, MODE, KB> sh;
  __shared__ __attribute__((aligned(16))) unsigned char lds_w[P::LDS_W];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int C = a.C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const int64_t step = gridDim.x;
  int64_t tile = blockIdx.x;

  // Gate parameters first, then the register phi tiles, the first x tile and
  // the LDS phi tiles (each wave stages its own blocks).
  const RawParam rp = load_gate_param<N, MODE>(a, tid);
  const auto wr = make_rsrc(a.phi_packed, (uint32_t)(N * NCB * P::NU) * 1024u);
  auto phi_off = [&](int u, int q, int i) -> uint32_t {
    const int cb = wave + kPersistWaves * q;
    return cb < NCB ? (uint32_t)(((i * NCB + cb) * P::NU + u) * 64 + lane) * 16u : kBufOob;
  };
  bf16x8_t wreg[KB][N][P::WR];
#pragma unroll
  for (int u = 0; u < P::NREG; ++u)
#pragma unroll
    for (int q = 0; q < KB; ++q)
#pragma unroll
      for (int i = 0; i < N; ++i) wreg[q][i][u] = __builtin_bit_cast(bf16x8_t, buf_load16(wr, phi_off(u, q, i)));
  U32x4 xa[KB][N];
  U32x4 xb[KB][N];
  split_load<N, KB, 0, KB>(xa, split_rsrc(a.x, tile, a.M, N * C), C, wave, lane);
  // Each LDS tile's blocks are loaded into registers together before any is
  // written: stored straight from each load, the writes made every load wait
  // for the one before (one register set reused: KB * N round trips a tile).
#pragma unroll
  for (int t = 0; t < P::NLDS; ++t) {
    U32x4 st[KB][N];
#pragma unroll
    for (int q = 0; q < KB; ++q)
#pragma unroll
      for (int i = 0; i < N; ++i) st[q][i] = buf_load16(wr, phi_off(P::NREG + t, q, i));
#pragma unroll
    for (int q = 0; q < KB; ++q)
#pragma unroll
      for (int i = 0; i < N; ++i)
        *reinterpret_cast<U32x4*>(lds_w + t * P::TILE_LDS + (((wave * KB + q) * N + i) * 64 + lane) * 16) = st[q][i];
  }
  if (tid < GateParams<N>::kCount) sh.prm[tid] = convert_param(rp, a.param_dtype);
  __syncthreads();  // gate parameters and LDS phi tiles visible

  // Pairs of steps (xa computes while xb loads, then the reverse), then the
  // leftover step; no exit between the steps of a pair (see pre_persist_kernel).
  const int64_t my_tiles = (ntiles - blockIdx.x + step - 1) / step;
  int64_t prev = -1;
  int slot = 0;
  int64_t k = 0;
  for (; k + 2 <= my_tiles; k += 2) {
    split_step<N, MODE, KB>(a, sh, xa, xb, wreg, lds_w, tile, prev, slot, tid, lane, wave);
    prev = tile;
    slot ^= 1;
    tile += step;
    split_step<N, MODE, KB>(a, sh, xb, xa, wreg, lds_w, tile, prev, slot, tid, lane, wave);
    prev = tile;
    slot ^= 1;
    tile += step;
  }
  if (k < my_tiles) {
    split_step<N, MODE, KB>(a, sh, xa, xb, wreg, lds_w, tile, prev, slot, tid, lane, wave);
    prev = tile;
    slot ^= 1;
  }
  if constexpr (MODE == kFull) {
    __syncthreads();  // the last tile's logits
    if (wave < P::SK_WAVES && a.h_res) split_sinkhorn<N>(a, sh.hres[slot ^ 1], prev, tid);
  }
}

}  // namespace mhc
