// Fused mHC pre phase for wide projections (n = 8): K-streamed MFMA.
//
// At n = 8, C = 768 the projection phi is [6144, 80] bf16 = 983 KB: it fits
// neither in a workgroup's registers and LDS (as it does at n = 4) nor does a
// 16-token x tile (192 KB) fit in registers next to it.  So phi streams from
// L2 and its cost is spread over a 32-token tile:
//   * one 8-wave workgroup per 32-token tile; wave w owns every 8th 32-column
//     chunk of the n*C row (K split 8 ways) for both 16-token M-blocks, so
//     each phi chunk is read once per tile and feeds two MFMAs;
//   * the K loop keeps D chunks in flight per wave: each chunk is two 16-byte
//     x loads (16 tokens x 32 columns per M-block, the MFMA A operands) and
//     NT 16-byte phi loads (the packed B operands, 16 output columns each);
//     v_mfma_f32_16x16x32_bf16 accumulates, bf16 dot2 forms the sum of
//     squares;
//   * the eight K-split partials meet in LDS.  The pre-aggregate's re-reads
//     of the tile's x (393 KB, from the Infinity Cache: it has left L2 by
//     then) need no result of the projection, so its first two rounds go out
//     before the partials are summed;
//   * 16 lanes per token then form inv_rms and the gates straight from the
//     partials: lane j takes mix j (h_pre for j < 8, h_post for 8 <= j < 16)
//     and the four h_res logits of row (j & 7), columns 4 * (j >> 3) .. + 3,
//     which is the layout the Sinkhorn iterations (sk8_*) run in, so h_res
//     never passes through LDS;
//   * the Sinkhorn iterations are spread between the pre-aggregate rounds:
//     VALU work while the next round's loads are in flight;
//   * with the RMSNorm epilogue the pre-aggregate chunks wait in LDS; after
//     the rounds 16 lanes per token sum their squares, and a last pass
//     scales, rounds and stores them.
// Arithmetic and rounding points as pre_persist_kernel, except x_norm: the
// MFMAs run on x and the fp32 result is scaled by inv_rms, the way the
// reference's fused kernel computes x_norm (model/mhc_fused.py:209-229), where
// the PyTorch path rounds x * inv_rms to bf16 before its GEMM (:845).  Rounding
// it here needs each row's sum of squares before the K loop, i.e. a second
// pass over the tile's 393 KB of x, which the tile cannot hold on chip.
//
// Reference semantics: model/mhc_fused.py:163-268, :533-559, :47-56;
// model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195.
#pragma once

#include "mhc_pre_persist.hpp"

namespace mhc {

constexpr int kKsWaves = 8;

template <int N, int MODE>
struct KsPlan {
  using S = PreShape<N, MODE>;
  static constexpr int FD = S::FD;
  static constexpr int NT = S::NT;
  static constexpr int G = N * N;
  static constexpr int WAVES = kKsWaves;
  static constexpr int MB = 2;             // 16-token M-blocks per tile (every wave)
  static constexpr int TM = 16 * MB;       // tokens per tile
  static constexpr int KS = WAVES;         // K split
  static constexpr int D = 3;              // chunks in flight per wave
  static constexpr int PB = 2;             // pre-aggregate items per lane per round (two rounds in flight)
  static_assert(N == 8, "16 lanes per token: mixes 0..2N-1 and half an 8 x 8 row each");
  static_assert(TM == WAVES * 4, "four tokens per wave");
};

template <int N, int MODE>
struct KsShared {
  using P = KsPlan<N, MODE>;
  alignas(16) float acc[P::KS][P::TM][P::FD];  // 16-byte reads of four h_res logits
  float ss[P::KS][P::TM];
  float prm[GateParams<N>::kCount];
  float hpre[P::TM][N];
};

// LDS of the RMSNorm epilogue: the tile's pre-aggregate, the gain (fp32) and
// each token's scale.
template <int N, int MODE, bool NORM>
struct KsNorm {
  using P = KsPlan<N, MODE>;
  static constexpr int kChunks = kMfmaMaxColBlocks * 4;  // 8-column chunks of a C <= 1024 row
  U32x4 stash[P::TM * kChunks];
  float gain[kMfmaMaxColBlocks * kCBlock];
  float scale[P::TM];
};
template <int N, int MODE>
struct KsNorm<N, MODE, false> {
  int unused;
};

template <int N, int MODE, bool NORM>
__global__ __launch_bounds__(kKsWaves * 64) void pre_kstream_kernel(PreArgs a) {
  using P = KsPlan<N, MODE>;
  using GP = GateParams<N>;
  using NS = KsNorm<N, MODE, NORM>;
  constexpr int FD = P::FD;
  constexpr int NT = P::NT;
  constexpr int TM = P::TM;
  constexpr int D = P::D;
  constexpr int T = P::WAVES * 64;
  static_assert(sizeof(KsShared<N, MODE>) + sizeof(NS) <= kLdsBytes, "LDS budget");
  __shared__ KsShared<N, MODE> sh;
  __shared__ NS nsh;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kq = wave;
  const int C = a.C;
  const int NC = N * C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const int NCH = N * NCB;                      // 32-column chunks in a row
  const int NJ = (NCH + P::KS - 1) / P::KS;     // chunks per wave (last ones may be empty)
  const int64_t M = a.M;
  const int64_t t0 = (int64_t)blockIdx.x * TM;
  const int valid = (int)(M - t0 < TM ? M - t0 : TM);

  const RawParam rp = load_gate_param<N, MODE>(a, tid);
  float gain[2] = {0.f, 0.f};  // norm gain of columns tid and tid + 512 (branch-free loads)
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * T;
      const float v = ld_any(a.norm_w, c < C ? c : 0, a.norm_dtype);
      gain[h] = c < C ? v : 0.f;
    }
  }

  // ---- K loop -----------------------------------------------------------
  const auto rx = make_rsrc(static_cast<const uint16_t*>(a.x) + t0 * NC, (uint32_t)valid * NC * 2u);
  const auto rw = make_rsrc(a.phi_packed, (uint32_t)(NCH * NT) * 1024u);
  const uint32_t xrow = (uint32_t)(r * NC) * 2u + (uint32_t)g * 16u;
  const uint32_t xblk = (uint32_t)(16 * NC) * 2u;  // offset of M-block 1
  U32x4 xs[D][P::MB];
  U32x4 ws[D][NT];
  // Workgroups walk their chunks in rotated orders, so the CUs of an XCD do
  // not all read the same few phi lines from the same L2 channels at once.
  const int rot = (int)(blockIdx.x % (unsigned)NJ);
  auto issue = [&](int slot_j, U32x4 (&xd)[P::MB], U32x4 (&wd)[NT]) {
    const int jr = slot_j < NJ ? (slot_j + rot < NJ ? slot_j + rot : slot_j + rot - NJ) : slot_j;
    const int k = kq + P::KS * jr;              // uniform
    const bool live = slot_j < NJ && k < NCH;
    const int i = live ? k / NCB : 0;
    const int cb = live ? k - i * NCB : 0;
    const int c0 = cb * kCBlock;
    const bool xl = live && c0 + g * 8 < C;
#pragma unroll
    for (int m = 0; m < P::MB; ++m)
      xd[m] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rx, (int)(xl ? xrow + m * xblk : kBufOob), (i * C + c0) * 2, 0));
    const uint32_t wo = live ? (uint32_t)lane * 16u : kBufOob;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      wd[nt] = __builtin_bit_cast(
          U32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)wo, (k * NT + nt) * 1024, 0));
  };
#pragma unroll
  for (int d = 0; d < D; ++d) issue(d, xs[d], ws[d]);

  f32x4_t acc[P::MB][NT];
  float ss[P::MB];
#pragma unroll
  for (int m = 0; m < P::MB; ++m) {
    ss[m] = 0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[m][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  for (int j0 = 0; j0 < NJ; j0 += D) {   // uniform trip count
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
      for (int m = 0; m < P::MB; ++m) {
        const U32x4 v = xs[d][m];
#pragma unroll
        for (int q = 0; q < 4; ++q) ss[m] = dot2_bf16(v.v[q], v.v[q], ss[m]);
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, v);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              av, __builtin_bit_cast(bf16x8_t, ws[d][nt]), acc[m][nt], 0, 0, 0);
      }
      issue(j0 + d + D, xs[d], ws[d]);
    }
  }
  // MFMA 16x16 result layout: lane l holds D[4*(l/16) + j][l % 16], j = 0..3.
#pragma unroll
  for (int m = 0; m < P::MB; ++m) {
    ss[m] += __shfl_xor(ss[m], 16, 64);
    ss[m] += __shfl_xor(ss[m], 32, 64);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      if (nt * 16 + r < FD)
#pragma unroll
        for (int j = 0; j < 4; ++j) sh.acc[kq][m * 16 + 4 * g + j][nt * 16 + r] = acc[m][nt][j];
    if (g == 0) sh.ss[kq][m * 16 + r] = ss[m];
  }
  if (tid < GP::kCount) sh.prm[tid] = convert_param(rp, a.param_dtype);
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) nsh.gain[tid + h * T] = gain[h];
  }

  // ---- pre-aggregate rounds --------------------------------------------------
  // Items are (token, 16-byte column chunk) pairs, PB per lane per round, in
  // two register buffers: rounds 0 and 1 are issued here, round r + 2 as soon
  // as round r is consumed.  A round past the end reads nothing (offsets out
  // of the descriptor) and stores nothing.
  constexpr int PB = P::PB;
  const int C8 = C / 8;
  const int items = TM * C8;
  const int nrounds = (items + PB * T - 1) / (PB * T);
  const auto rsub = make_rsrc(static_cast<uint16_t*>(a.sub_in) + t0 * C, (uint32_t)valid * C * 2u);
  auto pa_item = [&](int round, int b, int& tt, int& c) {
    const int p = (round * PB + b) * T + tid;
    tt = p < items ? p / C8 : TM;
    c = tt < TM ? (p - tt * C8) * 8 : 0;
  };
  auto pa_issue = [&](int round, U32x4 (&xv)[PB][N]) {
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      int tt, c;
      pa_item(round, b, tt, c);
      const uint32_t xo = tt < valid ? (uint32_t)(tt * NC + c) * 2u : kBufOob;
#pragma unroll
      for (int i = 0; i < N; ++i)
        xv[b][i] = buf_load16_nt(rx, xo, i * C * 2);  // x's last use in this launch
    }
  };
  auto pa_finish = [&](int round, const U32x4 (&xv)[PB][N]) {
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      int tt, c;
      pa_item(round, b, tt, c);
      const int ts = tt < TM ? tt : 0;
      uint32_t hlo[N];
      uint32_t hhi[N];
#pragma unroll
      for (int i = 0; i < N; ++i) {
        hlo[i] = pack_lo(sh.hpre[ts][i]);
        hhi[i] = pack_hi(sh.hpre[ts][i]);
      }
      const U32x4 pk = preagg_chunk<N>(xv[b], hlo, hhi);
      if constexpr (NORM) {
        if (tt < TM) nsh.stash[tt * NS::kChunks + (c >> 3)] = pk;
        continue;
      }
      // whole offset in the vector offset, scalar offset the literal 0 (see
      // persist_preagg: a 128-bit store reads its data registers after issue)
      buf_store16_nt(rsub, tt < valid ? (uint32_t)(tt * C + c) * 2u : kBufOob, pk);
    }
  };
  U32x4 xa[PB][N];
  U32x4 xb[PB][N];
  pa_issue(0, xa);
  pa_issue(1, xb);
  __syncthreads();  // partials and gate parameters visible

  // ---- inv_rms and gates: 16 lanes per token ----------------------------------
  const int tt = wave * 4 + (lane >> 4);
  const int jl = lane & 15;
  const int64_t tk = t0 + tt;
  const bool ok = tt < valid;
  float sq = 0.f;
#pragma unroll
  for (int w = 0; w < P::KS; ++w) sq += sh.ss[w][tt];
  const float inv = 1.0f / sqrtf(sq / (float)NC + a.rms_eps);
  if (jl == 0 && ok && a.inv_rms) a.inv_rms[tk] = inv;
  constexpr int NMIX = FD < 2 * N ? FD : 2 * N;  // pre (and post) mixes
  if (jl < NMIX) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < P::KS; ++w) sum += sh.acc[w][tt][jl];
    const float m = sum * inv;
    if (ok && a.mixes_raw) a.mixes_raw[tk * FD + jl] = m;
    // bias_pre[j] and bias_post[j - N] are adjacent: GP::kBiasPre + j for both
    const bool pre = jl < N;
    const float gs = gate_sigmoid(m, sh.prm[pre ? 0 : 1], sh.prm[GP::kBiasPre + jl], kBF16);
    const float h = pre ? round_to(__fadd_rn(gs, a.pre_eps), kBF16)   // gate_pre
                        : round_to(__fmul_rn(gs, a.post_mult), kBF16);  // gate_post
    if (pre) {
      sh.hpre[tt][jl] = h;
      if (ok && a.h_pre) st_any(a.h_pre, tk * N + jl, kBF16, h);
    } else if (ok) {
      st_any(a.h_post, tk * N + (jl - N), kBF16, h);
    }
  }
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  const int e0 = (jl & 7) * N + 4 * (jl >> 3);  // first of this lane's h_res entries
  if constexpr (MODE == kFull) {
    float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < P::KS; ++w) {
      const float4 pw = *reinterpret_cast<const float4*>(&sh.acc[w][tt][2 * N + e0]);
      s4[0] += pw.x;
      s4[1] += pw.y;
      s4[2] += pw.z;
      s4[3] += pw.w;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float m = s4[q] * inv;
      if (ok && a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e0 + q] = m;
      v[q] = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e0 + q], kBF16);
      if (ok && a.h_res_raw) st_any(a.h_res_raw, tk * P::G + e0 + q, kBF16, v[q]);
    }
  }
  __syncthreads();  // h_pre visible to every lane's pre-aggregate items

  // ---- Sinkhorn iterations between the pre-aggregate rounds ------------------
  const bool sk = MODE == kFull && a.h_res != nullptr;
  const int slots = (nrounds + 1) & ~1;  // rounds run in pairs
  const int sk_rest = a.sk_iters > 1 ? a.sk_iters - 1 : 0;
  int sk_done = 0;
  if (sk) sk8_start(v, a.sk_eps);
  auto sk_share = [&](int slot) {  // iterations due before slot's round is consumed
    if (!sk) return;
    const int target = (sk_rest * (slot + 1) + slots - 1) / slots;
    for (; sk_done < target; ++sk_done) sk8_iter(v, a.sk_eps);
  };
  for (int rd = 0; rd < nrounds; rd += 2) {  // uniform trip count, no exit between steps
    sk_share(rd);
    pa_finish(rd, xa);
    pa_issue(rd + 2, xa);
    sk_share(rd + 1);
    pa_finish(rd + 1, xb);
    pa_issue(rd + 3, xb);
  }
  if (sk && ok) {
#pragma unroll
    for (int q = 0; q < 4; ++q) st_any(a.h_res, tk * P::G + e0 + q, kBF16, v[q]);
  }
  if constexpr (NORM) {
    // RMSNorm over C: 16 lanes per token sum the squares of the stashed
    // (bf16-rounded) chunks jl, jl + 16, ...; then every item is scaled by
    // its token's 1 / sqrt(mean + norm_eps) and the gain, rounded, stored.
    __syncthreads();  // every chunk stashed
    float q2 = 0.f;
    for (int ch = jl; ch < C8; ch += 16) {
      const U32x4 pk = nsh.stash[tt * NS::kChunks + ch];
#pragma unroll
      for (int j = 0; j < 4; ++j) q2 = dot2_bf16(pk.v[j], pk.v[j], q2);
    }
    q2 = row_reduce<8, OpAdd>(q2);
    q2 = q2 + dpp_f<kDppRowMirror>(q2);
    if (jl == 0) nsh.scale[tt] = 1.0f / sqrtf(q2 / (float)C + a.norm_eps);
    __syncthreads();  // token scales visible
    for (int p = tid; p < items; p += T) {
      const int it = p / C8;
      const int c = (p - it * C8) * 8;
      const U32x4 pk = nsh.stash[it * NS::kChunks + (c >> 3)];
      const float sc = nsh.scale[it];
      const float4 w0 = *reinterpret_cast<const float4*>(&nsh.gain[c]);
      const float4 w1 = *reinterpret_cast<const float4*>(&nsh.gain[c + 4]);
      U32x4 y;
      y.v[0] = pack_bf16x2(bf16lo(pk.v[0]) * sc * w0.x, bf16hi(pk.v[0]) * sc * w0.y);
      y.v[1] = pack_bf16x2(bf16lo(pk.v[1]) * sc * w0.z, bf16hi(pk.v[1]) * sc * w0.w);
      y.v[2] = pack_bf16x2(bf16lo(pk.v[2]) * sc * w1.x, bf16hi(pk.v[2]) * sc * w1.y);
      y.v[3] = pack_bf16x2(bf16lo(pk.v[3]) * sc * w1.z, bf16hi(pk.v[3]) * sc * w1.w);
      buf_store16_nt(rsub, it < valid ? (uint32_t)(it * C + c) * 2u : kBufOob, y);
    }
  }
}

template <int N, int MODE>
hipError_t launch_pre_kstream_inst(const PreArgs& a, hipStream_t s) {
  constexpr int TM = KsPlan<N, MODE>::TM;
  const int64_t tiles = (a.M + TM - 1) / TM;
  if (a.norm_w)
    hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, true>), dim3((unsigned)tiles),
                       dim3(KsPlan<N, MODE>::WAVES * 64), 0, s, a);
  else
    hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false>), dim3((unsigned)tiles),
                       dim3(KsPlan<N, MODE>::WAVES * 64), 0, s, a);
  return hipGetLastError();
}

// n = 8 instances (mhc_pre_kstream_n8.hip).
hipError_t launch_pre_kstream_n8(const PreArgs& a, hipStream_t s);

}  // namespace mhc
