// Fused mHC pre phase for wide projections: K-streamed MFMA.
//
// Serves the shapes whose phi does not fit a workgroup's registers: n = 8 and
// n = 16 at any C, and n in {2, 4} at C > 1024.  At n = 8, C = 768 phi is
// [6144, 80] bf16 = 983 KB; neither it nor a 16-token x tile (192 KB) fits in
// registers next to the other.  So phi streams from L2 and its cost is spread
// over a token tile:
//   * one 8-wave workgroup per TM-token tile (32; 16 at n = 16).  Wave w owns
//     every KS-th 32-column chunk of the n*C row (K split KS ways) for all of
//     the tile's 16-token M-blocks, so each phi chunk is read once per tile and
//     feeds MB MFMAs.  KS = 8, except at n = 16 with H_res (18 output tiles of
//     16 columns): there two waves share each chunk, one per half of the output
//     tiles (KS = 4), so a wave's operands and accumulators stay in registers;
//   * a first pass over the wave's chunks forms each row's sum of squares
//     (bf16 dot2), so the projection can run on x_norm = bf16(x * inv_rms),
//     rounded as the PyTorch path rounds it (model/mhc_fused.py:845).  When
//     the kernel that wrote x handed its rows' sums over (PreArgs::x_ssq),
//     the pass is skipped and x is read twice, not three times;
//   * the K loop keeps D chunks in flight per wave: each chunk is MB 16-byte x
//     loads (16 tokens x 32 columns per M-block, the MFMA A operands) and NTW
//     16-byte phi loads (the packed B operands, 16 output columns each);
//     v_mfma_f32_16x16x32_bf16 accumulates;
//   * the K-split partials meet in LDS.  The pre-aggregate's re-reads of the
//     tile's x (from the Infinity Cache: it has left L2 by then) need no
//     result of the projection, so its first round goes out before the
//     partials are summed (and, but for bf16 at n >= 8, the second as well);
//   * LPT = 512 / TM lanes per token (16, or 32 at n = 16) then form inv_rms
//     and the gates straight from the partials: lane j takes mix j (h_pre for
//     j < n, h_post for n <= j < 2n) and its share of the n*n h_res logits in
//     the layout the Sinkhorn iterations run in (one element per lane for
//     n <= 4, half a row per lane, sk8_* / sk16_*, for n = 8 / 16), so h_res
//     never passes through LDS;
//   * the Sinkhorn iterations are spread between the pre-aggregate rounds:
//     VALU work while the next round's loads are in flight;
//   * with the RMSNorm epilogue (C <= 1024) the pre-aggregate chunks wait in
//     LDS; after the rounds the token's lanes sum their squares, and a last
//     pass scales, rounds and stores them.  Wider rows take a second launch
//     (the RMSNorm in place on the written sublayer input).
// Arithmetic and rounding points as pre_persist_kernel.  The tile's x is read
// three times (sums of squares, K loop, pre-aggregate; twice with x_ssq), the
// later reads mostly from the Infinity Cache.
//
// Reference semantics: model/mhc_fused.py:163-268, :533-559, :47-56;
// model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195.
#pragma once

#include "mhc_pre_persist.hpp"

namespace mhc {

constexpr int kKsWaves = 8;
constexpr int kKsNormMaxC = kMfmaMaxColBlocks * kCBlock;  // widest row of the fused RMSNorm

template <int N, int MODE>
struct KsPlan {
  using S = PreShape<N, MODE>;
  static constexpr int FD = S::FD;
  static constexpr int NT = S::NT;
  static constexpr int G = N * N;
  static constexpr int WAVES = kKsWaves;
  static constexpr int NH = NT > 9 ? 2 : 1;          // output-tile halves
  static constexpr int NTW = (NT + NH - 1) / NH;     // output tiles per wave
  static constexpr int KS = WAVES / NH;              // K split
  static constexpr int TM = N >= 16 ? 16 : 32;       // tokens per tile
  static constexpr int MB = TM / 16;                 // 16-token M-blocks (every wave)
  static constexpr int LPT = WAVES * 64 / TM;        // lanes per token in the gate phase
  static constexpr int TPW = 64 / LPT;               // tokens per wave
  static constexpr int D = 3;                        // chunks in flight per wave
  // pre-aggregate items per lane per round: one at n >= 8, where a round of
  // two (128 KB a workgroup at n = 8) issued at once held up the loop's tail
  // (C5 pre 52.5 -> 49.0 us with one, 48.6 us with the second round issued
  // after the gates); two at n <= 4 (C > 1024), where one measured level.
  static constexpr int PB = N >= 8 ? 1 : 2;
  static constexpr int SD = 4;                       // chunks in flight in the sums-of-squares pass
  static constexpr int SKV = G > LPT ? G / LPT : 1;  // Sinkhorn values per lane
  static constexpr int SKL = G / SKV;                // lanes holding distinct h_res values
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "n in {2, 4, 8, 16}");
  static_assert(2 * N <= LPT, "one pre / post mix per lane");
  static_assert(TM == WAVES * TPW, "whole tokens per wave");
  static_assert(SKV == 1 || SKV == 4 || SKV == 8, "Sinkhorn lane layouts");
  static_assert((KS & (KS - 1)) == 0, "power-of-two K split");
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
  static constexpr int kChunks = kKsNormMaxC / 8;  // 8-column chunks of a row
  U32x4 stash[P::TM * kChunks];
  float gain[kKsNormMaxC];
  float scale[P::TM];
};
template <int N, int MODE>
struct KsNorm<N, MODE, false> {
  int unused;
};

// Whether the fused RMSNorm epilogue fits beside the partials.
template <int N, int MODE>
constexpr bool ks_norm_fits() {
  return sizeof(KsShared<N, MODE>) + sizeof(KsNorm<N, MODE, true>) <= (size_t)kLdsBytes;
}

// First h_res entry of gate-phase lane jl (of P::SKV consecutive ones).
template <int N, int SKV>
__device__ __forceinline__ int ks_res_entry(int jl) {
  if constexpr (SKV == 1) return jl % (N * N);
  else if constexpr (SKV == 4) return (jl & 7) * N + 4 * (jl >> 3);  // n = 8: half row
  else return (jl >> 1) * N + 8 * (jl & 1);                           // n = 16: half row
}

// Sinkhorn on the gate-phase layout: first step (softmax, + eps, first column
// normalisation) and one more row + column normalisation.
template <int N, int SKV>
__device__ __forceinline__ void ks_sk_start(float (&v)[SKV], float eps) {
  if constexpr (SKV == 1) {
    const float mx = row_reduce<N, OpMax>(v[0]);
    const float e = expf(v[0] - mx);
    v[0] = e * __builtin_amdgcn_rcpf(row_reduce<N, OpAdd>(e)) + eps;
    v[0] = v[0] * __builtin_amdgcn_rcpf(col_sum<N>(v[0]) + eps);
  } else if constexpr (SKV == 4) {
    sk8_start(v, eps);
  } else {
    sk16_start(v, eps);
  }
}
template <int N, int SKV>
__device__ __forceinline__ void ks_sk_iter(float (&v)[SKV], float eps) {
  if constexpr (SKV == 1) {
    v[0] = v[0] * __builtin_amdgcn_rcpf(row_reduce<N, OpAdd>(v[0]) + eps);
    v[0] = v[0] * __builtin_amdgcn_rcpf(col_sum<N>(v[0]) + eps);
  } else if constexpr (SKV == 4) {
    sk8_iter(v, eps);
  } else {
    sk16_iter(v, eps);
  }
}

// Sum over the LPT lanes of one token (16: a DPP row; 32: two).
template <int LPT>
__device__ __forceinline__ float ks_token_sum(float q) {
  q = row_reduce<8, OpAdd>(q);
  q = q + dpp_f<kDppRowMirror>(q);
  if constexpr (LPT == 32) q = q + xor_lane16(q);
  return q;
}

// F32: fp32 stream and phi (the reference trainers' layout).  x_norm = x *
// inv_rms stays fp32 (the reference rounds it to the stream dtype) and is split
// into bf16 hi + lo MFMA operands, phi likewise (phi_packed holds the hi image
// of the packed layout, then the lo image); three products per pair (hi.hi,
// hi.lo, lo.hi) keep ~16 significant bits of each operand.  Gates, Sinkhorn
// output and the pre-aggregate are fp32 (products rounded, summed in stream
// order); the pre-aggregate items are 4-column chunks.  No fused norm (a
// second launch normalises in place).
constexpr bool kKsPairs = true;
// Chunk pairs (and fp32 whole-line x) at n in {2, 4, 8}; n = 16 splits the
// output tiles over two wave halves (several waves a K-split slot).
// pre_group_kernel follows the same chunk order at n = 8 (n <= 4 at
// C > 1024, the only n <= 4 shapes this kernel serves, have no group form).
template <int N, int MODE>
constexpr bool ks_pairs() {
  return kKsPairs && (N == 2 || N == 4 || N == 8);
}
// The wave's 4 KiB regroup block: its own partials slot (TM x FD fp32) where
// that is large enough (n = 8, full projection), else an LDS block of its own.
template <int N, int MODE>
constexpr bool ks_regroup_in_slot() {
  if constexpr (N == 2 || N == 4 || N == 8) {
    using P = KsPlan<N, MODE>;
    return P::TM * P::FD * 4 >= P::MB * 16 * 128;
  } else {
    return false;
  }
}

// PAIRS (bf16, n in {2, 4, 8}, C % 64 == 0): wave kq owns chunk pairs
// (2p, 2p + 1), p = kq + KS jr, 64 columns of one stream, contiguous in a
// token's row; each pair's x moves as whole 128-byte row pieces (8 rows x
// 128 B an instruction) and is regrouped into the MFMA A layout through a
// 4 KiB LDS block of the wave (its own partials slot sh.acc[kq], unused until
// the wave's K loop ends, at n = 8 with the full projection; else the norm
// stash or LDS of its own), where the operand layout reads 16 rows x 64 B,
// half of each line.
// The chunk order is 2p, 2p + 1 for the pair slots in rotated order;
// pre_group_kernel walks the same order.  C5 shape (8192 tokens, sums of
// squares handed over) 48.6 -> 43.3 us; the 64-token n = 8 group projection,
// which must follow the order, 12.7 -> 13.9 us (one box).  Wave kq taking a
// contiguous range of pairs instead measured the same at C5, slower at 64.
template <int N, int MODE, bool NORM, bool F32 = false, bool PAIRS = false>
__global__ __launch_bounds__(kKsWaves * 64) void pre_kstream_kernel(PreArgs a) {
  using P = KsPlan<N, MODE>;
  using GP = GateParams<N>;
  using NS = KsNorm<N, MODE, NORM>;
  static_assert(!(F32 && NORM), "fp32 streams: the norm runs as a second launch");
  static_assert(!PAIRS || (!F32 && ks_pairs<N, MODE>() && P::NH == 1), "chunk pairs: bf16, n in {2, 4, 8}");
  constexpr int FD = P::FD;
  constexpr int NT = P::NT;
  constexpr int NTW = P::NTW;
  constexpr int TM = P::TM;
  constexpr int D = F32 ? 2 : P::D;      // chunks in flight (fp32: hi and lo phi operands)
  constexpr int XQ = F32 ? 2 : 1;        // 16-byte loads per 8 columns of a row
  constexpr uint32_t ES = F32 ? 4u : 2u; // bytes per stream element
  constexpr int XDT = F32 ? kF32 : kBF16;
  constexpr int LPT = P::LPT;
  constexpr int SKV = P::SKV;
  constexpr int T = P::WAVES * 64;
  static_assert(sizeof(KsShared<N, MODE>) + sizeof(NS) <= kLdsBytes, "LDS budget");
  __shared__ KsShared<N, MODE> sh;
  __shared__ NS nsh;
  // Regroup blocks (4 KiB a wave) of the chunk pairs / whole-line fp32 x where
  // the partials slots are too small: the norm stash when there is one (it is
  // first written after the barrier that follows every wave's K loop), else
  // LDS of their own.
  constexpr bool kRgOut = (PAIRS || (F32 && N == 8)) && !ks_regroup_in_slot<N, MODE>();
  constexpr bool kRgOwn = kRgOut && !NORM;
  __shared__ __attribute__((aligned(16))) U32x4 s_rg[kRgOwn ? P::WAVES * P::MB * 128 : 1];
  static_assert(sizeof(KsShared<N, MODE>) + sizeof(NS) + sizeof(s_rg) <= kLdsBytes, "LDS budget (regroup)");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int kq = wave & (P::KS - 1);                  // K-split index
  const int nh = (int)((unsigned)wave / (unsigned)P::KS);  // half of the output tiles
  const int C = a.C;
  const int NC = N * C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const int NCH = N * NCB;                      // 32-column chunks in a row
  const int NJP = (NCH / 2 + P::KS - 1) / P::KS;  // PAIRS: pair slots per wave
  const int NJ = PAIRS ? 2 * NJP : (NCH + P::KS - 1) / P::KS;  // chunks per wave (last ones may be empty)
  const int64_t M = a.M;
  const int64_t t0 = (int64_t)blockIdx.x * TM;
  const int valid = (int)(M - t0 < TM ? M - t0 : TM);

  const RawParam rp = load_gate_param<N, MODE>(a, tid);
  // Sums of squares handed over by the kernel that wrote x (see PreArgs::
  // x_ssq): thread tt < TM sums row tt's partials in order.  Loaded before
  // the K loop's first chunks, so no wait on them.
  const bool given = a.x_ssq != nullptr;  // uniform
  float ss_given = 0.f;
  if (given && tid < TM && tid < valid) {
    const int P = C / kSsqCols;
    const float* src = a.x_ssq + (t0 + tid) * P;
    for (int j = 0; j < P; ++j) ss_given += src[j];
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

  // ---- K loop -----------------------------------------------------------
  const auto rx = make_rsrc(static_cast<const unsigned char*>(a.x) + t0 * NC * ES,
                            (uint32_t)valid * NC * ES);
  const uint32_t wimg = (uint32_t)(NCH * NT) * 1024u;  // bytes of one packed image
  const auto rw = make_rsrc(a.phi_packed, F32 ? 2u * wimg : wimg);
  const uint32_t xrow = (uint32_t)(r * NC) * ES + (uint32_t)g * 8u * ES;
  const uint32_t xblk = (uint32_t)(16 * NC) * ES;  // offset of M-block 1
  // x chunk k of every M-block (zeros past the row or past C).
  auto x_chunk = [&](int k, bool live, U32x4 (&xd)[P::MB][XQ]) {
    const int i = live ? k / NCB : 0;
    const int cb = live ? k - i * NCB : 0;
    const int c0 = cb * kCBlock;
    const bool xl = live && c0 + g * 8 < C;
#pragma unroll
    for (int m = 0; m < P::MB; ++m)
#pragma unroll
      for (int q = 0; q < XQ; ++q)
        xd[m][q] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rx, (int)(xl ? xrow + m * xblk + 16u * q : kBufOob),
                                                 (int)((i * C + c0) * ES), 0));
  };
  U32x4 xs[D][P::MB][XQ];
  U32x4 ws[D][NTW];
  U32x4 wl[F32 ? D : 1][NTW];  // lo phi operands (fp32)
  // Workgroups walk their chunks in rotated orders, so the CUs of an XCD do
  // not all read the same few phi lines from the same L2 channels at once.
  // Slot j of this wave is chunk kq + KS * ((j + rot) mod NJ); slots past NJ
  // read nothing.  At n = 16 phi (7 MB at C = 768) outgrows an XCD's 4 MB L2:
  // there every workgroup walks the same order, so the CUs of an XCD read each
  // phi line at about the same time and share its L2 fill (652 -> 553 us at
  // 16384 tokens; at n = 8 and at C = 2048 the rotation stays faster).
  const int NR = PAIRS ? NJP : NJ;  // slots the rotation turns (pair slots with PAIRS)
  const int rot = N == 16 ? 0 : (int)(blockIdx.x % (unsigned)NR);
  auto chunk_of = [&](int slot_j, bool& live) {
    if constexpr (PAIRS) {  // chunk slot_j of the sequence 2p, 2p + 1 over the rotated pair slots
      const int ps = slot_j >> 1;
      const int jr = ps < NJP ? (ps + rot < NJP ? ps + rot : ps + rot - NJP) : ps;
      const int pp = kq + P::KS * jr;  // uniform
      live = ps < NJP && 2 * pp < NCH;
      return 2 * pp + (slot_j & 1);
    }
    const int jr = slot_j < NJ ? (slot_j + rot < NJ ? slot_j + rot : slot_j + rot - NJ) : slot_j;
    const int k = kq + P::KS * jr;  // uniform
    live = slot_j < NJ && k < NCH;
    return k;
  };
  auto rg_block = [&]() -> U32x4* {
    if constexpr (kRgOwn) return &s_rg[wave * P::MB * 128];
    else if constexpr (kRgOut) {
      static_assert(!NORM || sizeof(nsh.stash) >= sizeof(U32x4) * P::WAVES * P::MB * 128, "regroup blocks in the stash");
      return &nsh.stash[wave * P::MB * 128];
    } else {
      return reinterpret_cast<U32x4*>(&sh.acc[kq][0][0]);
    }
  };
  // XROWS (fp32, n = 8): a chunk's 32 fp32 columns are one
  // 128-byte line of each row, loaded as whole lines (8 rows x 128 B an
  // instruction, XQ = 2 per M-block: lane row l / 8, 16-byte piece l % 8) and
  // regrouped into the operand layout through the wave's regroup block, as
  // the bf16 chunk pairs are; the operand layout's two loads
  // each read 16 rows x 64 B, half of every line.  The chunks, their order
  // and the MFMA inputs are unchanged.  fp32 C5 shape 107.4-109.3 -> 102.0-
  // 102.2 us (one box).
  constexpr bool XROWS = F32 && N == 8 && XQ == 2;  // n <= 4: 8 more VGPRs, one workgroup a CU fewer
  auto x_rows = [&](int k, bool live, U32x4 (&xd)[P::MB][XQ]) {
    const int i = live ? k / NCB : 0;
    const int c0 = live ? (k - i * NCB) * kCBlock : 0;
    const bool xl = live && c0 + 4 * (lane & 7) < C;
#pragma unroll
    for (int m = 0; m < P::MB; ++m)
#pragma unroll
      for (int u = 0; u < XQ; ++u)
        xd[m][u] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rx,
                                                 (int)(xl ? (uint32_t)((16 * m + 8 * u + (lane >> 3)) * NC) * ES +
                                                                16u * (lane & 7)
                                                          : kBufOob),
                                                 (int)((i * C + c0) * ES), 0));
  };
  // XROWS: a chunk's rows into the wave's regroup block and back, in place,
  // in the operand layout (xq: 16-byte piece 2g + xq of row r).
  auto rows_regroup = [&](U32x4 (&xd)[P::MB][XQ]) {
    U32x4* const rsb = rg_block();
#pragma unroll
    for (int m = 0; m < P::MB; ++m)
#pragma unroll
      for (int u = 0; u < XQ; ++u)
        rsb[(m * 16 + 8 * u + (lane >> 3)) * 8 + ((lane & 7) ^ ((lane >> 3) & 7))] = xd[m][u];
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int m = 0; m < P::MB; ++m)
#pragma unroll
      for (int q = 0; q < XQ; ++q) xd[m][q] = rsb[(m * 16 + r) * 8 + ((2 * g + q) ^ (r & 7))];
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  auto issue = [&](int slot_j, U32x4 (&xd)[P::MB][XQ], U32x4 (&wd)[NTW], U32x4 (&wdl)[NTW]) {
    bool live;
    const int k = chunk_of(slot_j, live);
    if constexpr (XROWS) x_rows(k, live, xd);
    else x_chunk(k, live, xd);
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int ntg = nh * NTW + nt;
      const int voff = (int)(live && ntg < NT ? (uint32_t)lane * 16u : kBufOob);
      wd[nt] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rw, voff, (k * NT + ntg) * 1024, 0));
      if constexpr (F32)
        wdl[nt] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rw, voff, (int)(wimg + (uint32_t)(k * NT + ntg) * 1024u), 0));
    }
  };
  // PAIRS: pair slot ps loads both chunks' phi operands and, per M-block,
  // the pair's 16 rows x 128 bytes as two instructions (lane: row l / 8 of 8,
  // 16-byte piece l % 8).
  constexpr int DP = 2;  // pairs in flight
  U32x4 xp[PAIRS ? DP : 1][PAIRS ? P::MB : 1][2];
  U32x4 wp[PAIRS ? DP : 1][2][PAIRS ? NTW : 1];
  auto load_pair_x = [&](int ps, U32x4 (&xd)[PAIRS ? P::MB : 1][2]) {
    bool live;
    const int k = chunk_of(2 * ps, live);  // the pair's first chunk
    const int i = live ? k / NCB : 0;
    const int c0 = live ? (k - i * NCB) * kCBlock : 0;
#pragma unroll
    for (int m = 0; m < (PAIRS ? P::MB : 1); ++m)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        xd[m][u] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rx,
                                                 (int)(live ? (uint32_t)((16 * m + 8 * u + (lane >> 3)) * NC) * ES +
                                                                  16u * (lane & 7)
                                                            : kBufOob),
                                                 (int)((i * C + c0) * ES), 0));
  };
  // The pair's rows into the wave's regroup block, and back in the operand
  // layout: chunk h of M-block m for this lane (row r, columns 8g .. + 7).
  auto pair_regroup = [&](const U32x4 (&xd)[PAIRS ? P::MB : 1][2], U32x4 (&ov)[2][PAIRS ? P::MB : 1]) {
    U32x4* const rsb = rg_block();
#pragma unroll
    for (int m = 0; m < (PAIRS ? P::MB : 1); ++m)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int rr = 8 * u + (lane >> 3);
        rsb[(m * 16 + rr) * 8 + ((lane & 7) ^ (rr & 7))] = xd[m][u];
      }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int m = 0; m < (PAIRS ? P::MB : 1); ++m) ov[h][m] = rsb[(m * 16 + r) * 8 + ((4 * h + g) ^ (r & 7))];
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  auto issue_pair = [&](int ps, U32x4 (&xd)[PAIRS ? P::MB : 1][2], U32x4 (&wd)[2][PAIRS ? NTW : 1]) {
    bool live;
    const int k = chunk_of(2 * ps, live);  // the pair's first chunk
    load_pair_x(ps, xd);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int nt = 0; nt < (PAIRS ? NTW : 1); ++nt)
        wd[h][nt] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rw, (int)(live ? (uint32_t)lane * 16u : kBufOob),
                                                  ((k + h) * NT + nt) * 1024, 0));
  };
  if constexpr (PAIRS) {
#pragma unroll
    for (int d = 0; d < DP; ++d) issue_pair(d, xp[d], wp[d]);
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, xs[d], ws[d], wl[F32 ? d : 0]);
  }

  // ---- sums of squares, then each row's inv_rms --------------------------------
  // A first pass over this wave's chunks in the K loop's order (SD in flight;
  // the K loop's first chunks are already out): lane (g, r) chains the dot2
  // squares of its 8 columns of row r, then the 16-lane groups are summed and
  // the K-split partials meet in LDS.  pre_group_kernel forms the same sums in
  // the same order.  At n = 16 the waves of the second output-tile half read
  // the same chunks as the first and skip the pass.
  float inv_r[P::MB];
  {
    float ss[P::MB];
#pragma unroll
    for (int m = 0; m < P::MB; ++m) ss[m] = 0.f;
    if (given) {  // uniform: the totals in slot 0, the other K-split slots zero
      if (tid < TM) sh.ss[0][tid] = ss_given;
      else if (tid < P::KS * TM) sh.ss[tid / TM][tid % TM] = 0.f;
    } else if constexpr (PAIRS) {  // the same chains, the pairs' x as row pieces (pair_regroup)
      for (int j0 = 0; j0 < NJP; j0 += P::SD / 2) {  // uniform trip count
        U32x4 xv[P::SD / 2][PAIRS ? P::MB : 1][2];
#pragma unroll
        for (int e = 0; e < P::SD / 2; ++e) load_pair_x(j0 + e, xv[e]);
#pragma unroll
        for (int e = 0; e < P::SD / 2; ++e) {
          U32x4 ov[2][PAIRS ? P::MB : 1];
          pair_regroup(xv[e], ov);
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int m = 0; m < P::MB; ++m)
#pragma unroll
              for (int q = 0; q < 4; ++q) ss[m] = dot2_bf16(ov[h][m].v[q], ov[h][m].v[q], ss[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < P::MB; ++m) {
        ss[m] += __shfl_xor(ss[m], 16, 64);
        ss[m] += __shfl_xor(ss[m], 32, 64);
        if (g == 0) sh.ss[kq][m * 16 + r] = ss[m];
      }
    } else if (P::NH == 1 || nh == 0) {  // uniform
      for (int j0 = 0; j0 < NJ; j0 += P::SD) {  // uniform trip count
        U32x4 v[P::SD][P::MB][XQ];
#pragma unroll
        for (int d = 0; d < P::SD; ++d) {
          bool live;
          const int k = chunk_of(j0 + d, live);
          if constexpr (XROWS) x_rows(k, live, v[d]);
          else x_chunk(k, live, v[d]);
        }
        if constexpr (XROWS) {
#pragma unroll
          for (int d = 0; d < P::SD; ++d) rows_regroup(v[d]);
        }
#pragma unroll
        for (int d = 0; d < P::SD; ++d)
#pragma unroll
          for (int m = 0; m < P::MB; ++m)
#pragma unroll
            for (int xq = 0; xq < XQ; ++xq)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                if constexpr (F32) {
                  const float f = __uint_as_float(v[d][m][xq].v[q]);
                  ss[m] = fmaf(f, f, ss[m]);
                } else {
                  ss[m] = dot2_bf16(v[d][m][xq].v[q], v[d][m][xq].v[q], ss[m]);
                }
              }
      }
#pragma unroll
      for (int m = 0; m < P::MB; ++m) {
        ss[m] += __shfl_xor(ss[m], 16, 64);
        ss[m] += __shfl_xor(ss[m], 32, 64);
        if (g == 0) sh.ss[kq][m * 16 + r] = ss[m];
      }
    }
    __syncthreads();  // sums of squares visible
#pragma unroll
    for (int m = 0; m < P::MB; ++m) {
      float sq = 0.f;
#pragma unroll
      for (int w = 0; w < P::KS; ++w) sq += sh.ss[w][m * 16 + r];
      inv_r[m] = 1.0f / sqrtf(sq / (float)NC + a.rms_eps);
    }
  }

  // ---- K loop: MFMAs on x_norm = bf16(x * inv_rms) ----------------------------
  f32x4_t acc[P::MB][NTW];
#pragma unroll
  for (int m = 0; m < P::MB; ++m)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) acc[m][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (PAIRS) {
    // the wave's regroup block, [M-block][row 16][16-byte slot 8], slots
    // swizzled by the row's low bits (conflict-free both ways): pair_regroup
    for (int j0 = 0; j0 < NJP; j0 += DP) {  // uniform trip count
#pragma unroll
      for (int d = 0; d < DP; ++d) {
        U32x4 ov[2][P::MB];
        pair_regroup(xp[d], ov);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int m = 0; m < P::MB; ++m) {
            const bf16x8_t av = __builtin_bit_cast(bf16x8_t, x_norm_chunk(ov[h][m], inv_r[m]));
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
              acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  av, __builtin_bit_cast(bf16x8_t, wp[d][h][nt]), acc[m][nt], 0, 0, 0);
          }
        issue_pair(j0 + d + DP, xp[d], wp[d]);
      }
    }
  }
  for (int j0 = 0; !PAIRS && j0 < NJ; j0 += D) {   // uniform trip count
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if constexpr (XROWS) rows_regroup(xs[d]);  // the chunk's rows into the operand layout
#pragma unroll
      for (int m = 0; m < P::MB; ++m) {
        if constexpr (F32) {  // fp32 x_norm split into hi + lo bf16 operands
          U32x4 h4, l4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x0 = __uint_as_float(xs[d][m][e >> 1].v[2 * (e & 1)]) * inv_r[m];
            const float x1 = __uint_as_float(xs[d][m][e >> 1].v[2 * (e & 1) + 1]) * inv_r[m];
            const uint32_t hp = pack_bf16x2(x0, x1);
            h4.v[e] = hp;
            l4.v[e] = pack_bf16x2(x0 - bf16lo(hp), x1 - bf16hi(hp));
          }
          const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, h4);
          const bf16x8_t al = __builtin_bit_cast(bf16x8_t, l4);
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) {
            const bf16x8_t bh = __builtin_bit_cast(bf16x8_t, ws[d][nt]);
            acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc[m][nt], 0, 0, 0);
            acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                ah, __builtin_bit_cast(bf16x8_t, wl[F32 ? d : 0][nt]), acc[m][nt], 0, 0, 0);
            acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc[m][nt], 0, 0, 0);
          }
        } else {
          const bf16x8_t av = __builtin_bit_cast(bf16x8_t, x_norm_chunk(xs[d][m][0], inv_r[m]));
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
            acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                av, __builtin_bit_cast(bf16x8_t, ws[d][nt]), acc[m][nt], 0, 0, 0);
        }
      }
      issue(j0 + d + D, xs[d], ws[d], wl[F32 ? d : 0]);
    }
  }
  // MFMA 16x16 result layout: lane l holds D[4*(l/16) + j][l % 16], j = 0..3.
#pragma unroll
  for (int m = 0; m < P::MB; ++m) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int ntg = nh * NTW + nt;
      if (ntg * 16 + r < FD)
#pragma unroll
        for (int j = 0; j < 4; ++j) sh.acc[kq][m * 16 + 4 * g + j][ntg * 16 + r] = acc[m][nt][j];
    }
  }
  if (tid < GP::kCount) sh.prm[tid] = convert_param(rp, a.param_dtype);
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * T;
      nsh.gain[c] = c < C ? word_elem(gain_w[h], c, a.norm_dtype) : 0.f;
    }
  }

  // ---- pre-aggregate rounds --------------------------------------------------
  // Items are (token, 16-byte column chunk) pairs, PB per lane per round, in
  // two register buffers: round 0 is issued here, round 1 here as well or,
  // with one item a round (bf16 at n >= 8), after the gates; round r + 2 as
  // soon as round r is consumed.  A round past the end reads nothing (offsets
  // out of the descriptor) and stores nothing.
  // (fp32: 4-column items, the same 16 bytes of each stream per item; two a
  // round, both rounds up front: C5 110.1 us against 112.0 us with one)
  constexpr int PB = F32 ? 2 : P::PB;
  constexpr bool kLateRound1 = PB == 1;
  constexpr int CW = F32 ? 4 : 8;  // columns per item
  const int C8 = C / CW;
  const int items = TM * C8;
  const int nrounds = (items + PB * T - 1) / (PB * T);
  const auto rsub = make_rsrc(static_cast<unsigned char*>(a.sub_in) + t0 * C * ES,
                              (uint32_t)valid * C * ES);
  auto pa_item = [&](int round, int b, int& tt, int& c) {
    const int p = (round * PB + b) * T + tid;
    tt = p < items ? p / C8 : TM;
    c = tt < TM ? (p - tt * C8) * CW : 0;
  };
  auto pa_issue = [&](int round, U32x4 (&xv)[PB][N]) {
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      int tt, c;
      pa_item(round, b, tt, c);
      const uint32_t xo = tt < valid ? (uint32_t)(tt * NC + c) * ES : kBufOob;
#pragma unroll
      for (int i = 0; i < N; ++i)
        xv[b][i] = buf_load16_nt(rx, xo, (int)(i * C * ES));  // x's last use in this launch
    }
  };
  auto pa_finish = [&](int round, const U32x4 (&xv)[PB][N]) {
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      int tt, c;
      pa_item(round, b, tt, c);
      const int ts = tt < TM ? tt : 0;
      if constexpr (F32) {  // products rounded to fp32, summed in stream order
        U32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < N; ++i)
            acc = __fadd_rn(acc, mul_nc(sh.hpre[ts][i], __uint_as_float(xv[b][i].v[e])));
          o.v[e] = __float_as_uint(acc);
        }
        buf_store16_nt(rsub, tt < valid ? (uint32_t)(tt * C + c) * ES : kBufOob, o);
        continue;
      }
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
      buf_store16_nt(rsub, tt < valid ? (uint32_t)(tt * C + c) * ES : kBufOob, pk);
    }
  };
  U32x4 xa[PB][N];
  U32x4 xb[PB][N];
  pa_issue(0, xa);
  if constexpr (!kLateRound1) pa_issue(1, xb);
  __syncthreads();  // partials and gate parameters visible

  // ---- inv_rms and gates: LPT lanes per token ---------------------------------
  const int tt = wave * P::TPW + lane / LPT;
  const int jl = lane % LPT;
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
    const float m = sum;  // the partials are already normalised
    if (ok && a.mixes_raw) a.mixes_raw[tk * FD + jl] = m;
    // bias_pre[j] and bias_post[j - N] are adjacent: GP::kBiasPre + j for both
    const bool pre = jl < N;
    const float gs = gate_sigmoid(m, sh.prm[pre ? 0 : 1], sh.prm[GP::kBiasPre + jl], XDT);
    const float h = pre ? round_to(__fadd_rn(gs, a.pre_eps), XDT)   // gate_pre
                        : round_to(mul_nc(gs, a.post_mult), XDT);  // gate_post
    if (pre) {
      sh.hpre[tt][jl] = h;
      if (ok && a.h_pre) st_any(a.h_pre, tk * N + jl, XDT, h);
    } else if (ok) {
      st_any(a.h_post, tk * N + (jl - N), XDT, h);
    }
  }
  float v[SKV];
#pragma unroll
  for (int q = 0; q < SKV; ++q) v[q] = 0.f;
  const int e0 = ks_res_entry<N, SKV>(jl);  // first of this lane's h_res entries
  const bool own = jl < P::SKL;             // n = 2: lanes past the 4 entries repeat them
  if constexpr (MODE == kFull) {
    float s[SKV];
#pragma unroll
    for (int q = 0; q < SKV; ++q) s[q] = 0.f;
#pragma unroll
    for (int w = 0; w < P::KS; ++w) {
      if constexpr (SKV == 1) {
        s[0] += sh.acc[w][tt][2 * N + e0];
      } else {
#pragma unroll
        for (int q4 = 0; q4 < SKV; q4 += 4) {
          const float4 pw = *reinterpret_cast<const float4*>(&sh.acc[w][tt][2 * N + e0 + q4]);
          s[q4 + 0] += pw.x;
          s[q4 + 1] += pw.y;
          s[q4 + 2] += pw.z;
          s[q4 + 3] += pw.w;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < SKV; ++q) {
      const float m = s[q];
      if (ok && own && a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e0 + q] = m;
      v[q] = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e0 + q], XDT);
      if (ok && own && a.h_res_raw) st_any(a.h_res_raw, tk * P::G + e0 + q, XDT, v[q]);
    }
  }
  __syncthreads();  // h_pre visible to every lane's pre-aggregate items
  if constexpr (kLateRound1) pa_issue(1, xb);

  // ---- Sinkhorn iterations between the pre-aggregate rounds ------------------
  const bool sk = MODE == kFull && a.h_res != nullptr;
  const int slots = (nrounds + 1) & ~1;  // rounds run in pairs
  const int sk_rest = a.sk_iters > 1 ? a.sk_iters - 1 : 0;
  int sk_done = 0;
  if (sk) ks_sk_start<N, SKV>(v, a.sk_eps);
  auto sk_share = [&](int slot) {  // iterations due before slot's round is consumed
    if (!sk) return;
    const int target = (sk_rest * (slot + 1) + slots - 1) / slots;
    for (; sk_done < target; ++sk_done) ks_sk_iter<N, SKV>(v, a.sk_eps);
  };
  for (int rd = 0; rd < nrounds; rd += 2) {  // uniform trip count, no exit between steps
    sk_share(rd);
    pa_finish(rd, xa);
    pa_issue(rd + 2, xa);
    sk_share(rd + 1);
    pa_finish(rd + 1, xb);
    pa_issue(rd + 3, xb);
  }
  if (sk && ok && own) {
#pragma unroll
    for (int q = 0; q < SKV; ++q) st_any(a.h_res, tk * P::G + e0 + q, XDT, v[q]);
  }
  if constexpr (NORM) {
    // RMSNorm over C: the token's LPT lanes sum the squares of the stashed
    // (bf16-rounded) chunks jl, jl + LPT, ...; then every item is scaled by
    // its token's 1 / sqrt(mean + norm_eps) and the gain, rounded, stored.
    __syncthreads();  // every chunk stashed
    float q2 = 0.f;
    for (int ch = jl; ch < C8; ch += LPT) {
      const U32x4 pk = nsh.stash[tt * NS::kChunks + ch];
#pragma unroll
      for (int j = 0; j < 4; ++j) q2 = dot2_bf16(pk.v[j], pk.v[j], q2);
    }
    q2 = ks_token_sum<LPT>(q2);
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
  const dim3 block(KsPlan<N, MODE>::WAVES * 64);
  if (a.x_dtype == kF32) {  // fp32 stream and phi: hi / lo operands, norm as a second launch
    if constexpr (N != 16) {
      PreArgs plain = a;
      plain.norm_w = nullptr;
      hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false, true>), dim3((unsigned)tiles), block, 0, s,
                         plain);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess || !a.norm_w) return e;
      return launch_expand_norm(a.sub_in, kF32, a.norm_w, a.norm_dtype, a.sub_in, a.M, 1, a.C,
                                a.norm_eps, s);
    }
    return hipErrorInvalidValue;
  }
  // chunk pairs where a pair's 64 columns lie in one stream (C % 64 == 0)
  const bool pairs = ks_pairs<N, MODE>() && a.C % 64 == 0;
  if (!a.norm_w) {
    if constexpr (ks_pairs<N, MODE>()) {
      if (pairs) {
        hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false, false, true>), dim3((unsigned)tiles), block, 0, s, a);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false>), dim3((unsigned)tiles), block, 0, s, a);
    return hipGetLastError();
  }
  if constexpr (ks_norm_fits<N, MODE>()) {
    if (a.C <= kKsNormMaxC) {
      if constexpr (ks_pairs<N, MODE>()) {
        if (pairs) {
          hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, true, false, true>), dim3((unsigned)tiles), block, 0, s, a);
          return hipGetLastError();
        }
      }
      hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, true>), dim3((unsigned)tiles), block, 0, s, a);
      return hipGetLastError();
    }
  }
  PreArgs plain = a;
  plain.norm_w = nullptr;
  if constexpr (ks_pairs<N, MODE>()) {
    if (pairs) hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false, false, true>), dim3((unsigned)tiles), block, 0, s, plain);
    else hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false>), dim3((unsigned)tiles), block, 0, s, plain);
  } else {
    hipLaunchKernelGGL((pre_kstream_kernel<N, MODE, false>), dim3((unsigned)tiles), block, 0, s, plain);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_expand_norm(a.sub_in, kBF16, a.norm_w, a.norm_dtype, a.sub_in, a.M, 1, a.C, a.norm_eps, s);
}

template <int N>
hipError_t launch_pre_kstream_mode(const PreArgs& a, hipStream_t s) {
  switch (a.mode) {
    case kFull: return launch_pre_kstream_inst<N, kFull>(a, s);
    case kNoHres: return launch_pre_kstream_inst<N, kNoHres>(a, s);
    case kHead: return launch_pre_kstream_inst<N, kHead>(a, s);
    default: return hipErrorInvalidValue;
  }
}

// Per-n instances (mhc_pre_kstream_n*.hip).
hipError_t launch_pre_kstream_n2(const PreArgs& a, hipStream_t s);
hipError_t launch_pre_kstream_n4(const PreArgs& a, hipStream_t s);
hipError_t launch_pre_kstream_n8(const PreArgs& a, hipStream_t s);
hipError_t launch_pre_kstream_n16(const PreArgs& a, hipStream_t s);

}  // namespace mhc
