// Pre phase for small batches on MFMA: one workgroup per group of G tokens
// (G a power of two, at most 16), phi streamed from L2.  bf16 streams, packed
// phi, n in {1, 2, 4, 8}, C <= 1024, C % 8 == 0.
//
// At decode sizes the large-batch kernels leave most of the chip idle: the
// persistent kernel (n <= 4) puts one 16-token tile on each of a handful of
// CUs, each of which first pulls the whole of phi into registers, and the
// K-streamed kernel (n = 8) one 32-token tile per workgroup.  Here M / G
// workgroups each run a single MFMA tile with only G of its 16 rows live:
//   * wave w walks the 32-column blocks the same wave of the large-batch
//     kernel walks, in the same order (pre_persist_kernel's for n <= 4;
//     pre_kstream_kernel's, with its per-tile rotation, for n = 8).  The MFMA
//     accumulation chains, the per-wave sums of squares and the cross-wave
//     sums are then the large-batch kernel's, so every output is bit for bit
//     what that kernel writes and the results do not depend on the batch size;
//   * each block is one A-operand load (lanes of rows past the group read
//     nothing) and NT B-operand loads of the packed phi image (1 KiB per wave
//     instruction, padding columns skipped), with P blocks in flight per wave;
//   * the A operands of the live rows go to LDS as they are consumed, so the
//     pre-aggregate runs one column pair per lane over the whole workgroup
//     instead of on the few lanes that hold a live row;
//   * gates take one (token, feature) per thread; the Sinkhorn runs on the
//     last waves with the large-batch kernel's lane layout (sinkhorn_lane<N>
//     for n <= 4, the half-row sk8_* layout for n = 8), before their share of
//     the pre-aggregate;
//   * the RMSNorm epilogue sums its squares in the large-batch kernel's order.
// Rounding points as pre_persist_kernel.
//
// Reference semantics: model/mhc_fused.py:163-268, :533-559, :47-56;
// model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195.
#pragma once

#include "mhc_pre_kstream.hpp"

namespace mhc {

constexpr int kGrpWaves = 8;
constexpr int kKsTileTokens = 32;  // tokens of one pre_kstream_kernel tile (its rotation key)

template <int N, int MODE, int KB>
struct GroupPlan {
  using S = PreShape<N, MODE>;
  static constexpr int FD = S::FD;
  static constexpr int NT = S::NT;
  static constexpr int NN = N * N;
  static constexpr int LAST_COLS = FD - 16 * (NT - 1);  // real columns of the last tile
  static constexpr int NB = N * KB;                     // 32-column blocks per wave, at most
  // phi blocks in flight per wave: NT registers of 4 VGPRs a block, at most
  // 40 such registers (28 for the wide n = 8 projection at C > 512, whose
  // accumulators and Sinkhorn need the rest).
  static constexpr int PMAX = (NT >= 4 && KB >= 3 ? 28 : 40) / NT;
  static constexpr int P = NB < PMAX ? NB : PMAX;
  static constexpr bool KS_ORDER = N == 8;
  static constexpr int CMAX = 256 * KB;
  static constexpr int ROW = N * CMAX + 8;  // LDS x row in bf16 elements, 16 bytes of pad
  static constexpr int GFIT = 98304 / (2 * ROW);
  static constexpr int GLDS = GFIT >= 16 ? 16 : GFIT >= 8 ? 8 : GFIT >= 4 ? 4 : GFIT >= 2 ? 2 : 1;
  // A group's h_pre fits one wave, one (token, stream) per lane.
  static constexpr int GMAX = GLDS * N <= 64 ? GLDS : 64 / N;
  // 16-byte x chunks per lane for the group's rows (row-contiguous loads).
  static constexpr int XW = (GMAX * N * CMAX / 8 + kGrpWaves * 64 - 1) / (kGrpWaves * 64);
  static constexpr int SKL = N == 8 ? 16 : NN;  // Sinkhorn lanes per token
  static constexpr int SK_TOK = 64 / SKL;       // tokens per Sinkhorn wave
};

template <int N, int MODE, int KB, bool NORM>
struct GroupShared {
  using P = GroupPlan<N, MODE, KB>;
  float prm[GateParams<N>::kCount];
  alignas(16) float acc[kGrpWaves][16][P::FD];  // per-wave partial projections of the live rows
  float ss[kGrpWaves][16];                      // per-wave partial sums of squares
  U32x4 zero;                                   // A operand of rows past the group
  float hw[kGrpWaves][64];                      // each wave's copy of the group's h_pre
  alignas(16) uint16_t xs[P::GMAX][P::ROW];     // the group's x rows
  // RMSNorm epilogue: rounded pre-aggregate, gain, square-sum partials, scales.
  uint32_t ys[NORM ? P::GMAX : 1][NORM ? P::CMAX / 2 : 1];
  float gain[NORM ? P::CMAX : 1];
  float q2[NORM ? P::GMAX : 1][32];
  float scale[16];
};

// PH: 0 = the whole pre phase; 1 and 2 = the two launches of the split form
// (launch_pre_group_split): 1 = the projection of output tile blockIdx.y only,
// its finished mixes (the cross-wave sums) parked as fp32 in the first FD * 4
// bytes of each token's sublayer-input row; 2 = everything else, the mixes
// read back from there (before any sublayer input is stored).
template <int N, int MODE, int KB, bool NORM, int PH = 0>
__global__ __launch_bounds__(kGrpWaves * 64) void pre_group_kernel(PreArgs a, int G, int row_ss) {
  using P = GroupPlan<N, MODE, KB>;
  using GP = GateParams<N>;
  static_assert(PH != 1 || !NORM, "the projection launch has no norm");
  constexpr int FD = P::FD;
  constexpr int NT = P::NT;
  constexpr int NTL = PH == 1 ? 1 : NT;     // output tiles this launch projects
  constexpr int PB = PH == 1 ? (P::NB < 24 ? P::NB : 24) : P::P;  // blocks in flight per wave
  constexpr int NN = P::NN;
  constexpr int T = kGrpWaves * 64;
  static_assert(sizeof(GroupShared<N, MODE, KB, NORM>) <= kLdsBytes, "LDS budget");
  static_assert(P::CMAX <= 2 * T, "two gain columns per thread");
  __shared__ GroupShared<N, MODE, KB, NORM> sh;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int C = a.C;
  const int NC = N * C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const int NCH = N * NCB;                              // 32-column blocks of a row
  const int NJ = (NCH + kGrpWaves - 1) / kGrpWaves;     // blocks per wave, kstream order
  const int64_t t0 = wave_uniform((int64_t)blockIdx.x * G);
  const int valid = (int)(a.M - t0 < G ? a.M - t0 : G);
  const int nt0 = PH == 1 ? (int)blockIdx.y : 0;  // first output tile projected here
  // Mixes parked in the sublayer-input rows between the two split launches.
  float* const park = static_cast<float*>(a.sub_in);
  const int64_t park_row = (int64_t)C / 2;  // floats per sublayer-input row
  // pre_kstream_kernel rotates each tile's block order by (tile % NJ), or,
  // with its chunk pairs (C % 64 == 0), the pair slots by (tile % (NJ / 2)).
  const bool pairs = P::KS_ORDER && ks_pairs<N, MODE>() && C % 64 == 0;  // uniform
  const int NJP = NJ / 2;  // pair slots per wave (NJ = C / 32 is even then)
  const int rot = P::KS_ORDER ? (int)((t0 / kKsTileTokens) % (pairs ? NJP : NJ)) : 0;

  const RawParam rp = load_gate_param<N, MODE>(a, tid);
  // Sums of squares handed over by the kernel that wrote x, used where the
  // large-batch kernel uses them (n = 8: pre_kstream_kernel), summed in the
  // same order, so the two stay bit-identical.
  const bool given = P::KS_ORDER && a.x_ssq != nullptr;  // uniform
  float ss_given = 0.f;
  if (given && tid < G && tid < valid) {
    const int PS = C / kSsqCols;
    const float* src = a.x_ssq + (t0 + tid) * PS;
    for (int j = 0; j < PS; ++j) ss_given += src[j];
  }
  // norm gain words of columns tid and tid + T, converted where they are
  // stored to LDS (ld_any's per-dtype branch made the prologue's loads wait)
  uint32_t gain_w[2] = {0u, 0u};
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * T;
      gain_w[h] = ld_word(a.norm_w, C, c < C ? c : 0, a.norm_dtype);
    }
  }

  // ---- x rows: row-contiguous loads (1 KiB per wave instruction), first ----
  // 16-byte chunk j of the group's rows (they are contiguous in memory) is
  // lane j % 64 of instruction j / 64; instruction (u, wave) = u * 8 + wave.
  const int NC8 = NC / 8;
  const int nchunk = G * NC8;
  const auto rx = make_rsrc(static_cast<const uint16_t*>(a.x) + t0 * NC, (uint32_t)valid * NC * 2u);
  U32x4 xl[P::XW];
#pragma unroll
  for (int u = 0; u < P::XW; ++u) {
    const int j = (u * kGrpWaves + wave) * 64 + lane;
    xl[u] = buf_load16_nt(rx, j < nchunk ? (uint32_t)j * 16u : kBufOob, 0);
  }

  // ---- phi blocks, P in flight per wave ---------------------------------------
  const auto rw = make_rsrc(a.phi_packed, (uint32_t)(NCH * NT) * 1024u);
  // Block b of this wave: stream i, column block cb; false past the row.
  auto block_of = [&](int b, int& i, int& cb) -> bool {
    if constexpr (P::KS_ORDER) {
      int k;
      bool live;
      if (pairs) {  // chunks 2p, 2p + 1 of the rotated pair slots, p = wave + 8 jr
        const int ps = b >> 1;
        const int jr = ps < NJP ? (ps + rot < NJP ? ps + rot : ps + rot - NJP) : ps;
        const int pp = wave + kGrpWaves * jr;
        k = 2 * pp + (b & 1);
        live = ps < NJP && 2 * pp < NCH;
      } else {
        const int jr = b < NJ ? (b + rot < NJ ? b + rot : b + rot - NJ) : b;
        k = wave + kGrpWaves * jr;
        live = b < NJ && k < NCH;
      }
      i = live ? k / NCB : 0;
      cb = live ? k - i * NCB : 0;
      return live;
    } else {
      i = b % N;
      cb = wave + kGrpWaves * (b / N);
      return cb < NCB;
    }
  };
  U32x4 wq[PH == 2 ? 1 : PB][NTL];
  auto issue = [&](int b) {
    int i, cb;
    const bool live = block_of(b, i, cb);
#pragma unroll
    for (int u = 0; u < NTL; ++u) {
      const int nt = nt0 + u;
      const bool pad = nt == NT - 1 && r >= P::LAST_COLS;
      wq[b % PB][u] = buf_load16(
          rw, live && !pad ? (uint32_t)(((i * NCB + cb) * NT + nt) * 64 + lane) * 16u : kBufOob);
    }
  };
  if constexpr (PH != 2) {
#pragma unroll
    for (int b = 0; b < PB; ++b) issue(b);
  } else {
    // The parked mixes into partial slot 0 (the other slots are not read).
    for (int idx = tid; idx < G * FD; idx += T) {
      const int tt = idx / FD;
      const int f = idx - tt * FD;
      sh.acc[0][tt][f] = tt < valid ? park[(t0 + tt) * park_row + f] : 0.f;
    }
  }

  // x rows into LDS (waits for the x loads only: they were issued first).
#pragma unroll
  for (int u = 0; u < P::XW; ++u) {
    const int j = (u * kGrpWaves + wave) * 64 + lane;
    if (j < nchunk) {
      const int t = j / NC8;
      *reinterpret_cast<U32x4*>(&sh.xs[t][(j - t * NC8) * 8]) = xl[u];
    }
  }
  if (tid == 0) sh.zero = U32x4{{0u, 0u, 0u, 0u}};
  if (tid < GP::kCount) sh.prm[tid] = convert_param(rp, a.param_dtype);
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (tid + h * T < P::CMAX) {
        const int c = tid + h * T;
        sh.gain[c] = c < C ? word_elem(gain_w[h], c, a.norm_dtype) : 0.f;
      }
  }
  __syncthreads();  // x rows, zero block and parameters visible

  // ---- projection: MFMA over this wave's blocks --------------------------------
  // Lane (g, r) of block b: row r, columns c0 + 8g .. + 7 of stream i; zeros
  // past the group's rows or past C.
  auto a_of = [&](int b) -> U32x4 {
    int i, cb;
    const bool live = block_of(b, i, cb);
    const int c0 = cb * kCBlock;
    const U32x4* src = live && r < G && c0 + g * 8 < C
                           ? reinterpret_cast<const U32x4*>(&sh.xs[r][i * C + c0 + 8 * g])
                           : &sh.zero;
    return *src;
  };
  const float nc = (float)NC;
  auto inv_of = [&](int tt) {
    float sq = 0.f;
#pragma unroll
    for (int w = 0; w < kGrpWaves; ++w) sq += sh.ss[w][tt];
    return 1.0f / sqrtf(sq / nc + a.rms_eps);
  };
  // The projection runs on x_norm = bf16(x * inv_rms), rounded as the
  // reference rounds it (model/mhc_fused.py:845), so the sums of squares come
  // first (in the large-batch kernel's order), then a barrier, then the MFMAs.
  if (given) {  // uniform: the totals in slot 0, the other waves' slots zero
    if (tid < G) sh.ss[0][tid] = ss_given;
    else if (tid < kGrpWaves * 16 && tid % 16 < G && tid >= 16) sh.ss[tid / 16][tid % 16] = 0.f;
  } else if (row_ss) {  // uniform
    // The row-staged persistent kernel's order (persist_row_sumsq): lane l
    // chains the row's chunks at bytes 16 l + 1024 k (the row is a whole
    // number of 1 KiB pieces) in k order, then the wave butterfly.  The total
    // goes to ss[0], the other waves' partials are zero.
    for (int t = wave; t < G; t += kGrpWaves) {  // uniform
      float s = 0.f;
      for (int k = 0; k < NC / 512; ++k) {
        const U32x4 v = *reinterpret_cast<const U32x4*>(&sh.xs[t][k * 512 + lane * 8]);
#pragma unroll
        for (int j = 0; j < 4; ++j) s = dot2_bf16(v.v[j], v.v[j], s);
      }
      s = wave_sum(s);
      if (lane == 0) sh.ss[0][t] = s;
    }
    if (wave > 0 && g == 0 && r < G) sh.ss[wave][r] = 0.f;
  } else {
    float ss = 0.f;
#pragma unroll
    for (int b = 0; b < P::NB; ++b) {
      const U32x4 v = a_of(b);
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = dot2_bf16(v.v[j], v.v[j], ss);
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (g == 0 && r < G) sh.ss[wave][r] = ss;
  }
  __syncthreads();  // sums of squares (and parked mixes) visible
  if constexpr (PH != 2) {
    const float inv_r = inv_of(r < G ? r : 0);
    f32x4_t acc[NTL];
#pragma unroll
    for (int u = 0; u < NTL; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < P::NB; ++b) {
      const bf16x8_t av = __builtin_bit_cast(bf16x8_t, x_norm_chunk(a_of(b), inv_r));
#pragma unroll
      for (int u = 0; u < NTL; ++u)
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, wq[b % PB][u]),
                                                         acc[u], 0, 0, 0);
      if (b + PB < P::NB) issue(b + PB);
    }
    // MFMA 16x16 result layout: lane l holds D[4*(l/16) + j][l % 16], j = 0..3.
#pragma unroll
    for (int u = 0; u < NTL; ++u) {
      const int nt = nt0 + u;
      if (nt * 16 + r < FD)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (4 * g + j < G) sh.acc[wave][4 * g + j][nt * 16 + r] = acc[u][j];
    }
    __syncthreads();  // partials visible
  }
  if constexpr (PH == 1) {
    // The cross-wave sums of this tile's 16 columns, in wave order from zero
    // (the sum the gates below form), parked for the second launch.
    for (int idx = tid; idx < G * 16; idx += T) {
      const int tt = idx >> 4;
      const int f = nt0 * 16 + (idx & 15);
      if (tt < valid && f < FD) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kGrpWaves; ++w) sum += sh.acc[w][tt][f];
        park[(t0 + tt) * park_row + f] = sum;
      }
    }
    return;
  }

  // ---- gates straight from the partials, no further barrier ------------------
  // (the partials are already normalised).
  auto mix_of = [&](int tt, int f, float) {
    if constexpr (PH == 2) return sh.acc[0][tt][f];  // parked: the same sum
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kGrpWaves; ++w) sum += sh.acc[w][tt][f];
    return sum;
  };
  // Every wave: h_pre of the group's tokens, lane = (token, stream).
  const int sk_waves = MODE == kFull && a.h_res ? (G + P::SK_TOK - 1) / P::SK_TOK : 0;
  const int post_wave = kGrpWaves - 1 - sk_waves;  // writes h_pre / h_post / inv / mixes
  float hp = 0.f;
  {
    const int tt = lane / N;
    const int i = lane % N;
    if (tt < G) {
      const float inv = inv_of(tt);
      const float m = mix_of(tt, i, inv);
      hp = gate_pre(m, sh.prm[0], sh.prm[GP::kBiasPre + i], a.pre_eps, kBF16);
      if (wave == post_wave && tt < valid) {
        const int64_t tk = t0 + tt;
        if (a.h_pre) st_any(a.h_pre, tk * N + i, kBF16, hp);
        if (a.inv_rms && i == 0) a.inv_rms[tk] = inv;
        if (a.mixes_raw) a.mixes_raw[tk * FD + i] = m;
        if constexpr (MODE != kHead) {
          const float mp = mix_of(tt, N + i, inv);
          st_any(a.h_post, tk * N + i, kBF16,
                 gate_post(mp, sh.prm[1], sh.prm[GP::kBiasPost + i], a.post_mult, kBF16));
          if (a.mixes_raw) a.mixes_raw[tk * FD + N + i] = mp;
        }
      }
    }
  }

  // The wave's own copy in LDS for the pre-aggregate items (a lane-indexed
  // shuffle there would read zeros from lanes that ran out of items).  A
  // wave's LDS accesses complete in order, so no barrier is needed.
  sh.hw[wave][lane] = hp;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // The last waves: h_res logits of their tokens, then the Sinkhorn, before
  // their share of the pre-aggregate.
  if constexpr (MODE == kFull) {
    const int sw = kGrpWaves - 1 - wave;  // uniform
    if (sw < sk_waves) {
      const int tt = sw * P::SK_TOK + lane / P::SKL;
      const int ts = tt < G ? tt : 0;
      const bool ok = tt < valid;
      const int64_t tk = t0 + tt;
      const float inv = inv_of(ts);
      if constexpr (N == 8) {
        const int jl = lane & 15;
        const int e0 = (jl & 7) * N + 4 * (jl >> 3);  // row (jl & 7), columns 4 (jl >> 3) ..
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float m = mix_of(ts, 2 * N + e0 + q, inv);
          v[q] = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e0 + q], kBF16);
          if (ok && a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e0 + q] = m;
          if (ok && a.h_res_raw) st_any(a.h_res_raw, tk * NN + e0 + q, kBF16, v[q]);
        }
        sk8_start(v, a.sk_eps);
        for (int it = 1; it < a.sk_iters; ++it) sk8_iter(v, a.sk_eps);
        if (ok) {
#pragma unroll
          for (int q = 0; q < 4; ++q) st_any(a.h_res, tk * NN + e0 + q, kBF16, v[q]);
        }
      } else {
        const int e = lane % NN;
        const float m = mix_of(ts, 2 * N + e, inv);
        const float h = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e], kBF16);
        if (ok && a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e] = m;
        if (ok && a.h_res_raw) st_any(a.h_res_raw, tk * NN + e, kBF16, h);
        const float v = sinkhorn_lane<N>(h, a.sk_iters, a.sk_eps);
        if (ok) st_any(a.h_res, tk * NN + e, kBF16, v);
      }
    } else if (!a.h_res && wave == post_wave) {
      // No Sinkhorn wanted: the raw logits (and their mixes) still go out.
      for (int idx = lane; idx < G * NN; idx += 64) {
        const int tt = idx / NN;
        const int e = idx - tt * NN;
        if (tt < valid) {
          const int64_t tk = t0 + tt;
          const float m = mix_of(tt, 2 * N + e, inv_of(tt));
          if (a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e] = m;
          if (a.h_res_raw) st_any(a.h_res_raw, tk * NN + e, kBF16, gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e], kBF16));
        }
      }
    }
  }

  // ---- pre-aggregate: one column pair per item -------------------------------
  const int C2 = C / 2;
  const int items = G * C2;
  const auto rsub = make_rsrc(static_cast<uint16_t*>(a.sub_in) + t0 * C, (uint32_t)valid * C * 2u);
  for (int idx = tid; idx < items; idx += T) {
    const int tt = idx / C2;
    const int d = idx - tt * C2;
    uint32_t xd[N];
    uint32_t hlo[N];
    uint32_t hhi[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      xd[i] = *reinterpret_cast<const uint32_t*>(&sh.xs[tt][i * C + 2 * d]);
      const float h = sh.hw[wave][tt * N + i];
      hlo[i] = pack_lo(h);
      hhi[i] = pack_hi(h);
    }
    const uint32_t y = preagg_pair<N>(xd, hlo, hhi);
    if constexpr (NORM) {
      sh.ys[tt][d] = y;
    } else {
      __builtin_amdgcn_raw_buffer_store_b32(y, rsub, tt < valid ? (tt * C + 2 * d) * 2 : (int)kBufOob,
                                            0, kNt);
    }
  }

  // ---- RMSNorm over C: squares summed in the large-batch kernel's order ------
  if constexpr (NORM) {
    __syncthreads();  // the rounded pre-aggregate complete
    if constexpr (!P::KS_ORDER) {
      // pre_persist_kernel: lane (g, r) of wave w chains the chunks at columns
      // (w + 8q) * 32 + 8g over q; then (g0 + g1) + (g2 + g3), then over w.
      for (int idx = tid; idx < G * 32; idx += T) {
        const int tt = idx >> 5;
        const int w = (idx >> 2) & 7;
        const int gg = idx & 3;
        float q = 0.f;
#pragma unroll
        for (int qb = 0; qb < KB; ++qb) {
          const int c0 = (w + kGrpWaves * qb) * kCBlock + 8 * gg;
          if (c0 < C) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t y = sh.ys[tt][c0 / 2 + j];
              q = dot2_bf16(y, y, q);
            }
          }
        }
        sh.q2[tt][idx & 31] = q;
      }
      __syncthreads();
      if (tid < G) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kGrpWaves; ++w)
          t += (sh.q2[tid][4 * w] + sh.q2[tid][4 * w + 1]) + (sh.q2[tid][4 * w + 2] + sh.q2[tid][4 * w + 3]);
        sh.scale[tid] = 1.0f / sqrtf(t / (float)C + a.norm_eps);
      }
    } else {
      // pre_kstream_kernel: 16 lanes per token chain the chunks jl, jl + 16, ..,
      // then an 8-lane butterfly and the row mirror.
      const int tt = wave * 4 + (lane >> 4);
      const int ts = tt < G ? tt : 0;
      const int jl = lane & 15;
      float q = 0.f;
      for (int ch = jl; ch < C / 8; ch += 16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t y = sh.ys[ts][4 * ch + j];
          q = dot2_bf16(y, y, q);
        }
      }
      q = row_reduce<8, OpAdd>(q);
      q = q + dpp_f<kDppRowMirror>(q);
      if (jl == 0 && tt < G) sh.scale[tt] = 1.0f / sqrtf(q / (float)C + a.norm_eps);
    }
    __syncthreads();  // token scales visible
    for (int idx = tid; idx < items; idx += T) {
      const int tt = idx / C2;
      const int d = idx - tt * C2;
      const uint32_t y = sh.ys[tt][d];
      const float sc = sh.scale[tt];
      const uint32_t o = pack_bf16x2(bf16lo(y) * sc * sh.gain[2 * d], bf16hi(y) * sc * sh.gain[2 * d + 1]);
      __builtin_amdgcn_raw_buffer_store_b32(o, rsub, tt < valid ? (tt * C + 2 * d) * 2 : (int)kBufOob,
                                            0, kNt);
    }
  }
}

// Tokens per workgroup: enough workgroups for one per CU, as a power of two
// no larger than the LDS allows.
template <int N, int MODE, int KB>
int group_tokens(int64_t M, int num_cus) {
  int G = 1;
  while (G < GroupPlan<N, MODE, KB>::GMAX && (int64_t)G * num_cus < M) G *= 2;
  return G;
}

template <int N, int MODE, int KB>
hipError_t launch_pre_group_inst(const PreArgs& a, int num_cus, hipStream_t s) {
  const int G = group_tokens<N, MODE, KB>(a.M, num_cus);
  const int64_t grid = (a.M + G - 1) / G;
  // Sum the squares in the order of the large-batch kernel this shape would
  // run: row order where launch_pre_persist_inst picks row staging.
  int row_ss = 0;
  if constexpr (N <= 4) {
    if constexpr (PersistRow<N, MODE, KB>::OK)
      row_ss = !a.norm_w && a.C == 256 * KB && pre_row_staging() ? 1 : 0;
  }
  if (a.norm_w)
    hipLaunchKernelGGL((pre_group_kernel<N, MODE, KB, true>), dim3((unsigned)grid),
                       dim3(kGrpWaves * 64), 0, s, a, G, row_ss);
  else
    hipLaunchKernelGGL((pre_group_kernel<N, MODE, KB, false>), dim3((unsigned)grid),
                       dim3(kGrpWaves * 64), 0, s, a, G, row_ss);
  return hipGetLastError();
}

// The split form (n = 8, bf16): the projection of each group's 16-column
// output tiles on NT workgroups of their own (each streams 1 / NT of phi from
// L2 instead of all of it: one workgroup's phi stream is bound by its CU's
// vector-memory path), the mixes parked in the sublayer-input rows, then a
// second launch for the gates, the Sinkhorn, the pre-aggregate and the norm.
// The same MFMA chains and cross-wave sums as the one-launch kernel, so the
// results are bit for bit the same.  Needs FD fp32 values to fit a bf16 row
// of C (4 FD <= 2 C).
template <int N, int MODE, int KB>
hipError_t launch_pre_group_split_inst(const PreArgs& a, int num_cus, hipStream_t s) {
  using P = GroupPlan<N, MODE, KB>;
  int G1 = 1;  // projection groups: enough workgroups (groups x NT) for one per CU
  while (G1 < P::GMAX && ((a.M + G1 - 1) / G1) * P::NT > num_cus) G1 *= 2;
  const int64_t grid1 = (a.M + G1 - 1) / G1;
  hipLaunchKernelGGL((pre_group_kernel<N, MODE, KB, false, 1>), dim3((unsigned)grid1, P::NT),
                     dim3(kGrpWaves * 64), 0, s, a, G1, 0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int G = group_tokens<N, MODE, KB>(a.M, num_cus);
  const int64_t grid = (a.M + G - 1) / G;
  if (a.norm_w)
    hipLaunchKernelGGL((pre_group_kernel<N, MODE, KB, true, 2>), dim3((unsigned)grid),
                       dim3(kGrpWaves * 64), 0, s, a, G, 0);
  else
    hipLaunchKernelGGL((pre_group_kernel<N, MODE, KB, false, 2>), dim3((unsigned)grid),
                       dim3(kGrpWaves * 64), 0, s, a, G, 0);
  return hipGetLastError();
}

template <int N, int MODE, int... KBS>
hipError_t dispatch_group_kb(const PreArgs& a, int kb, int num_cus, hipStream_t s) {
  hipError_t r = hipErrorInvalidValue;
  bool done = false;
  const bool split = N == 8 && a.M <= pre_group_split_tokens() &&
                     4 * PreShape<N, MODE>::FD <= 2 * a.C;
  if (split) {
    ((!done && KBS >= kb ? (r = launch_pre_group_split_inst<N, MODE, KBS>(a, num_cus, s), done = true)
                         : false),
     ...);
    return r;
  }
  ((!done && KBS >= kb ? (r = launch_pre_group_inst<N, MODE, KBS>(a, num_cus, s), done = true) : false),
   ...);
  return r;
}

template <int N>
hipError_t dispatch_group_mode(const PreArgs& a, int num_cus, hipStream_t s) {
  const int kb = persist_kb_needed(a.C);
  switch (a.mode) {
    case kFull: return dispatch_group_kb<N, kFull, 1, 2, 3, 4>(a, kb, num_cus, s);
    case kNoHres: return dispatch_group_kb<N, kNoHres, 1, 2, 3, 4>(a, kb, num_cus, s);
    case kHead:
      if constexpr (N > 1) return dispatch_group_kb<N, kHead, 1, 2, 3, 4>(a, kb, num_cus, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

// Per-n entry points (mhc_pre_group_n*.hip).
hipError_t launch_pre_group_n1(const PreArgs& a, int num_cus, hipStream_t s);
hipError_t launch_pre_group_n2(const PreArgs& a, int num_cus, hipStream_t s);
hipError_t launch_pre_group_n4(const PreArgs& a, int num_cus, hipStream_t s);
hipError_t launch_pre_group_n8(const PreArgs& a, int num_cus, hipStream_t s);

}  // namespace mhc
