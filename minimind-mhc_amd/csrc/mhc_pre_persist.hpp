// Persistent fused mHC pre phase on MFMA, bf16 streams (gfx950).
//
// Per token, with x read from HBM exactly once:
//   ss        = sum_k x[k]^2                    (fp32, bf16 dot2 on the held registers)
//   inv_rms   = 1 / sqrt(ss / (n*C) + rms_eps)
//   xn[k]     = bf16(x[k] * inv_rms)            (the reference's x_norm, rounded to the
//                                                stream dtype: model/mhc_fused.py:845)
//   mixes[f]  = sum_k xn[k] * phi[k, f]         (v_mfma_f32_16x16x32_bf16, fp32 accumulate)
//   gates     h_pre = sigmoid(a_pre*m + b_pre) + pre_eps
//             h_post = post_mult * sigmoid(a_post*m + b_post)
//             h_res_raw = a_res*m + b_res
//             each op rounded to bf16 as the reference's torch ops round it
//   h_res     = Sinkhorn(h_res_raw) in fp32     (one matrix element per lane)
//   sub_in[c] = sum_i bf16(h_pre[i] * x[i*C + c])
// The token tile's n*C row is split over the waves by 32-column blocks, so
// each wave holds all n streams of its columns and the pre-aggregate (a sum
// over streams at a fixed column) is wave-local.  Scheduled for HBM:
//   * one 8-wave workgroup per CU walks the 16-token tiles blockIdx.x,
//     blockIdx.x + gridDim.x, ... until the tiles run out;
//   * wave w owns the 32-column blocks cb = w, w + 8, ... of every stream;
//   * phi stays resident for the workgroup's lifetime as MFMA B operands: the
//     first NREG 16-column tiles in registers, the next NLDS tiles in LDS (the
//     last, partial tile stored compactly: lanes past its real columns read a
//     shared zero block), any rest re-read from L2 per tile.  At n=4, C=768
//     all of phi (96 VGPRs a lane) lives in registers and the MFMAs read no
//     memory at all;
//   * x tiles are DEPTH-buffered in registers.  The loads of tile t+DEPTH go
//     out chunk by chunk while tile t's pre-aggregate frees its registers, so
//     load issue overlaps the VALU work instead of stalling all waves at once;
//   * with row staging (ROW; C == 256 * KB, phi in registers, no norm) the
//     in-flight tile is loaded as whole-row 1 KiB pieces instead of in the
//     MFMA operand layout, and at the start of its step goes through LDS
//     (one more barrier a tile) into the operand registers: the operand
//     layout's loads split every 128-byte line between two waves, which
//     streams ~20% slower;
//   * x loads and sub_in stores are raw buffer ops bounded by a per-tile
//     descriptor: missing tokens / columns are zero-filled (or dropped) by
//     hardware, so no load sits behind a branch and the compiler waits only
//     for the tile it is about to use;
//   * x loads and sub_in stores carry the non-temporal cache policy with the
//     device-scope bit (each byte is touched once per launch);
//   * the tile loop issues no other global load: the vector-memory counter
//     retires in order, so waiting on any load issued after a prefetch would
//     also wait for the prefetch.  Gate scalars and biases are read once, with
//     branch-free loads issued before everything else, and kept in LDS as fp32.
//
// Per tile, two workgroup barriers:
//   0. all waves: partial sums of squares of the tile's rows -> LDS (with row
//      staging: each wave's two whole rows, from the row-layout registers,
//      beside the tile's copy into LDS);
//   -- barrier --
//   1. all waves: inv_rms of each row, x_norm, MFMA partial projections -> LDS
//      (two slots, alternating per tile, so a fast wave may start the next
//      tile's partials while others still read this tile's);
//   -- barrier --
//   2. waves 0..SK_WAVES-1 first run the Sinkhorn-Knopp iterations of the
//      PREVIOUS tile (h_res logits from the other LDS slot): a ~20-step
//      dependent chain that overlaps the VALU-heavy pre-aggregate of the wave
//      sharing the SIMD;
//   3. every wave computes the tile's h_pre itself (one (token, stream) per
//      lane, straight from the partials, then spread to the lanes that use it)
//      and runs its pre-aggregate; one wave also writes h_post / h_pre /
//      inv_rms, and the gate waves write the h_res logits (one per lane) for
//      the next tile's Sinkhorn.
// The next tile's x loads go out in three batches along the way.  The last
// tile's Sinkhorn runs after the loop.
//
// Reference semantics: model/mhc_fused.py:163-268, :533-559, :47-56,
// :820-830; model/mhc_fused_no_hres.py:48-145; model/mhc_common.py:128-195.
#pragma once

#include "mhc_internal.hpp"

namespace mhc {

// Projection width per mode and its 16-wide MFMA column tiles.
template <int N, int MODE>
struct PreShape {
  static constexpr int FD = MODE == kFull ? 2 * N + N * N : (MODE == kNoHres ? 2 * N : N);
  static constexpr int NT = (FD + 15) / 16;
};

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
  float acc[2][kPersistWaves][kTokTile][FD];  // per-wave partial projections, 2 slots
  float ss[2][kPersistWaves][kTokTile];       // per-wave partial sums of squares
  float hres[2][kTokTile * N * N];            // h_res logits, two tiles in flight
  U32x4 zero;                                 // B operand of padding columns
};

// LDS of the optional RMSNorm epilogue: each tile's pre-aggregate waits in LDS
// (lane-private slots, two tiles) until the next tile's barrier has made every
// wave's sum-of-squares partial visible; the gain lives in LDS as fp32.
template <bool NORM, int KB>
struct PersistNorm {
  static constexpr int kChunks = kPersistWaves * KB * 4;  // 8-column chunks per token row
  U32x4 stash[2][kTokTile * kChunks];                     // [slot][token][chunk]
  float gain[kMfmaMaxColBlocks * kCBlock];
  float ss2[2][kPersistWaves][kTokTile];                  // per-wave partials, 2 slots
};
template <int KB>
struct PersistNorm<false, KB> {
  int unused;
};

template <int N, int MODE, int KB, bool NORM = false>
struct PersistPlan {
  using S = PreShape<N, MODE>;
  static constexpr int FD = S::FD;
  static constexpr int NT = S::NT;
  static constexpr int G = N * N;
  static constexpr int LAST_COLS = FD - 16 * (NT - 1);  // real columns of the last tile
  // Registers: two x buffers (the tile being computed and the next one, whose
  // loads go out in small batches during the current step) and as many whole
  // phi tiles as fit in the rest of the budget (the other ~60 VGPRs are
  // working set); phi tiles that do not fit are read from LDS each tile.
  static constexpr int XTILE = KB * N * 4;  // VGPRs of one x tile (and of one phi tile)
  // With the norm epilogue one x tile's worth less: its stores and the stash
  // traffic need working registers inside the tile loop.
  static constexpr int kRegBudget = (XTILE <= 48 ? 192 : 160) - (NORM ? XTILE : 0);
  static constexpr int DEPTH = 2;
  static constexpr int REG_LEFT = kRegBudget - DEPTH * XTILE;
  static constexpr int REG_FIT = REG_LEFT > 0 ? REG_LEFT / XTILE : 0;
  static constexpr int NREG = REG_FIT < NT ? REG_FIT : NT;
  // LDS: shared scratch, then phi tiles NREG.. while they fit
  static constexpr int SHARED = (int)sizeof(PersistShared<N, FD>) + (int)sizeof(PersistNorm<NORM, KB>);
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
  // The first x tile's loads go out before the LDS phi tiles are written when
  // the staging registers of those tiles fit beside it.
  static constexpr bool X_EARLY = (NREG + NLDS + 1) * XTILE <= 224;
  // Column blocks of the next tile loaded at the three points of a step:
  // [0, B1) at its start, [B1, B2) after the first barrier, [B2, KB) after the
  // second.  Spreading the loads keeps a steady ~32 KiB per CU in flight; a
  // whole tile issued at once overflows the CU's request queue and stalls the
  // issuing waves.
  static constexpr int B1 = (KB + 2) / 3;
  static constexpr int B2 = (2 * KB + 2) / 3;
  // Waves that run the Sinkhorn (whole waves covering a tile's TM*G elements);
  // the gates run on the others.  Without h_res every wave runs the gates.
  static constexpr int SK_WAVES = MODE == kFull ? (kTokTile * G + 63) / 64 : 0;
  static constexpr int GATE_LANES = (kPersistWaves - SK_WAVES) * 64;
  static_assert(SK_WAVES < kPersistWaves, "gates need at least one wave");
  static_assert(2 * SK_WAVES <= kPersistWaves, "the last two Sinkhorns run side by side");
  static_assert(kTokTile * N <= 64, "one wave holds a tile's h_pre, one per lane");
  static_assert(kPersistWaves * kTokTile * FD * 4 >= 64 * 16, "partials area doubles as a write sink");
  // Wave that writes h_post (and h_pre / inv_rms when asked for).
  static constexpr int POST_WAVE = kPersistWaves - 1;
};

// Row staging of x (C == 256 * KB, phi wholly in registers, no norm epilogue).
// A 16-token tile is loaded with row-contiguous 1 KiB wave loads (lane l reads
// 16 bytes at l * 16 of a 1 KiB piece of the tile), written to LDS, and read
// back in the MFMA operand layout.  The operand layout's own loads put 16 rows
// x 64 bytes in each wave instruction (every 128-byte line split between two
// waves); on MI355X that pattern streams at ~4.8 TB/s where whole rows stream
// at ~6.1 TB/s.  Wave w loads pieces w * PW .. w * PW + PW - 1 (PW = n * KB, as
// many 16-byte chunks a lane as the operand layout holds), into the same
// registers the operand layout used for the in-flight tile.
template <int N, int MODE, int KB>
struct PersistRow {
  using P = PersistPlan<N, MODE, KB, false>;
  static constexpr int NC = N * KB * 256;              // n * C
  static constexpr int RCH = NC / 8;                   // 16-byte chunks of a token row
  static constexpr int PW = N * KB;                    // 1 KiB pieces per wave
  static constexpr int BYTES = kTokTile * NC * 2;      // the tile in LDS
  static constexpr int SCH = KB * 32;                  // 16-byte chunks of a sublayer-input row
  // The sublayer input goes out through LDS as whole rows (persist_stage_store)
  // where that measured faster (MI355X, 16384 tokens: n = 1, C = 1024 20.1 ->
  // 16.5 us; n = 2, C = 768 20.1 -> 19.3; n = 4, C = 256 at 65536 tokens 52.3
  // -> 50.9).  At n * KB = 8 it measured level (n = 2, C = 1024) or slower
  // (n = 4, C = 512: 22.5 -> 23.1); at 12 (n = 4, C = 768) the kernel already
  // holds 192 VGPRs of phi and x tiles and the staging spilled.
  static constexpr bool STAGE = N * KB <= 6;
  static constexpr int SUBB = STAGE ? kTokTile * SCH * 16 : 0;  // the tile's sublayer input in LDS
  // Load batches [0,R1) [R1,R2) [R2,PW) at three points of a step.  The
  // second (after the first barrier) carries half the tile: measured on MI355X
  // at C2 (PW = 12), splits 4/8/12 -> 4/10/12 took the pre launch from
  // 30.0-31.3 to 29.6 us; 4/9, 3/9 and 5/10 measured the same, 4/11 slower.
  static constexpr int R1 = (PW + 2) / 3;
  static constexpr int R2 = 5 * PW / 6;
  // A row is a whole number of 1 KiB pieces (n * KB even), so each wave holds
  // two whole rows and every lane the same columns of both (persist_row_sumsq).
  static constexpr bool OK = P::NREG == P::NT && RCH % 16 == 0 && (NC * 2) % 1024 == 0 &&
                             P::SHARED + 256 + BYTES + SUBB <= kLdsBytes;
};

// LDS byte of 16-byte chunk j of token row t.  The chunk index is XORed with
// the row's low 4 bits: the operand-layout reads (16 rows at one column, the
// rows 6 KiB apart) then hit 16 different 16-byte bank groups, and a row-
// contiguous write still covers whole aligned 256-byte groups.
template <int RCH>
__device__ __forceinline__ uint32_t row_lds_off(int t, int j) {
  return (uint32_t)(t * RCH + (j ^ (t & 15))) * 16u;
}

// Pieces [P0, P1) of this wave's share of a tile into xn (flat chunk p is
// xn[p / N][p % N]).  A token past the end reads zeros (bounded descriptor).
template <int N, int MODE, int KB, int P0, int P1>
__device__ __forceinline__ void persist_load_row(U32x4 (&xn)[KB][N], __amdgpu_buffer_rsrc_t rsrc,
                                                 int wave, int lane) {
  using RW = PersistRow<N, MODE, KB>;
#pragma unroll
  for (int p = P0; p < P1; ++p)
    xn[p / N][p % N] = buf_load16_nt<kNtSc1>(rsrc, (uint32_t)lane * 16u, (wave * RW::PW + p) * 1024);
}

// Row pieces [P0, P1) of the next tile, issued a share at a time from inside a
// compute loop over KB column blocks: at(q) issues the q-th share.  Loads
// spread through the step keep a steady amount in flight; a batch issued at
// once stalls the issuing wave on the CU's full request queue, and one
// issued at the end of a step leaves its latency exposed at the next.
template <int N, int MODE, int KB, int P0, int P1>
struct RowIssue {
  U32x4 (&xn)[KB][N];
  __amdgpu_buffer_rsrc_t rn;
  int wave, lane;
  __device__ __forceinline__ void at(int q) const {
    using RW = PersistRow<N, MODE, KB>;
    constexpr int PER = (P1 - P0 + KB - 1) / KB;
#pragma unroll
    for (int p = P0; p < P1; ++p)
      if (p >= P0 + q * PER && p < P0 + (q + 1) * PER)
        xn[p / N][p % N] = buf_load16_nt<kNtSc1>(rn, (uint32_t)lane * 16u, (wave * RW::PW + p) * 1024);
  }
};
struct NoIssue {
  __device__ __forceinline__ void at(int) const {}
};

// This wave's row pieces [P0, P1) of a tile -> LDS.
template <int N, int MODE, int KB, int P0, int P1>
__device__ __forceinline__ void persist_row_to_lds(unsigned char* xl, const U32x4 (&xn)[KB][N],
                                                   int wave, int lane) {
  using RW = PersistRow<N, MODE, KB>;
#pragma unroll
  for (int p = P0; p < P1; ++p) {
    const int J = (wave * RW::PW + p) * 64 + lane;  // chunk of the tile
    const int t = J / RW::RCH;
    *reinterpret_cast<U32x4*>(xl + row_lds_off<RW::RCH>(t, J - t * RW::RCH)) = xn[p / N][p % N];
  }
}

// The operand layout of this wave's column blocks from LDS: lane (r, g) of
// block q, stream i holds row r, columns c0 + 8g .. c0 + 8g + 7.
template <int N, int MODE, int KB>
__device__ __forceinline__ void persist_lds_to_operands(const unsigned char* xl, U32x4 (&xr)[KB][N],
                                                        int wave, int lane) {
  using RW = PersistRow<N, MODE, KB>;
  constexpr int C = KB * 256;
  const int r = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int q = 0; q < KB; ++q)
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int j = (i * C + (wave + kPersistWaves * q) * kCBlock) / 8 + g;
      xr[q][i] = *reinterpret_cast<const U32x4*>(xl + row_lds_off<RW::RCH>(r, j));
    }
}

// Tokens of a tile that exist (0 for a tile past the end).
__device__ __forceinline__ int tile_tokens(int64_t tile, int64_t ntiles, int64_t M) {
  if (tile >= ntiles) return 0;
  const int64_t left = M - tile * kTokTile;
  return left < kTokTile ? (int)left : kTokTile;
}

// Buffer descriptor over one tile's x rows: valid * n*C * 2 bytes (no records
// for a tile past the end, so its loads read zeros without touching memory).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_tile_rsrc(const uint16_t* __restrict__ x,
                                                              int64_t tile, int64_t ntiles,
                                                              int64_t M, int NC) {
  const int valid = tile_tokens(tile, ntiles, M);
  return make_rsrc(x + (valid > 0 ? tile * kTokTile * (int64_t)NC : 0),
                   (uint32_t)valid * (uint32_t)NC * 2u);
}

// Column part of the lane offset for column block q of this wave: lane (r, g)
// reads row r, columns c0 + 8g .. c0 + 8g + 7 (the row part is added by the
// caller).  A column block past C gets kBufOob (reads zeros).  For loads the
// per-stream offset travels in the scalar offset.
__device__ __forceinline__ uint32_t x_lane_off(int q, int wave, int g, int C) {
  const int c0 = (wave + kPersistWaves * q) * kCBlock;
  return c0 + g * 8 < C ? (uint32_t)g * 16u : kBufOob;
}

// Load column blocks [Q0, Q1) of this lane's x chunks of one tile.
template <int N, int KB, int Q0, int Q1>
__device__ __forceinline__ void persist_load_part(U32x4 (&xr)[KB][N], __amdgpu_buffer_rsrc_t rsrc,
                                                  int C, int wave, int r, int g) {
  const uint32_t row_off = (uint32_t)(r * N * C) * 2u;
#pragma unroll
  for (int q = Q0; q < Q1; ++q) {
    const int c0 = (wave + kPersistWaves * q) * kCBlock;
    const uint32_t lo = x_lane_off(q, wave, g, C);
    const uint32_t voff = lo == kBufOob ? kBufOob : row_off + lo;
#pragma unroll
    for (int i = 0; i < N; ++i)
      xr[q][i] = buf_load16_nt<kNtSc1>(rsrc, voff, (i * C + c0) * 2);
  }
}

// ---- phase 0: this wave's partial sums of squares of the tile's rows -> LDS.
// Lane (r, g) adds its chunks of row r in (block, stream) order, the four
// lanes of a row are summed by a butterfly, and the eight waves' partials are
// added in wave order (persist_inv_rms): every pre kernel that must agree bit
// for bit with this one (pre_group_kernel) sums in this order.
template <int N, int FD, int KB>
__device__ __forceinline__ void persist_sumsq(PersistShared<N, FD>& sh, const U32x4 (&xr)[KB][N], int slot,
                                              int lane, int wave) {
  const int r = lane & 15;
  const int g = lane >> 4;
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < KB; ++q)
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = dot2_bf16(xr[q][i].v[j], xr[q][i].v[j], ss);
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if (g == 0) sh.ss[slot][wave][r] = ss;
}

// ---- row staging, phase 0: the sums of squares of this wave's two rows.
// The tile arrives in row layout: wave w holds rows 2w and 2w + 1 as pieces
// [0, PW/2) and [PW/2, PW) of 1 KiB, lane l holding bytes 16 l .. 16 l + 15 of
// each piece.  Lane l chains the dot2 squares of its chunks of each row in
// piece order, a wave butterfly (wave_sum) adds the lanes, and lane 0 writes
// the totals to ss[slot][0][row].  ss[slot][1..7] hold zeros (set at launch),
// so persist_inv_rms adds each total to zeros: exact.  pre_group_kernel sums
// in this order when the persistent kernel would stage rows.
template <int N, int MODE, int KB, int FD>
__device__ __forceinline__ void persist_row_sumsq(PersistShared<N, FD>& sh, const U32x4 (&xn)[KB][N],
                                                  int slot, int wave, int lane) {
  using RW = PersistRow<N, MODE, KB>;
  static_assert(RW::PW % 2 == 0, "whole pieces per row");
  float s0 = 0.f;
  float s1 = 0.f;
#pragma unroll
  for (int p = 0; p < RW::PW; ++p) {
    const U32x4 v = xn[p / N][p % N];
    float& s = p < RW::PW / 2 ? s0 : s1;  // compile-time after unrolling
#pragma unroll
    for (int j = 0; j < 4; ++j) s = dot2_bf16(v.v[j], v.v[j], s);
  }
  s0 = wave_sum(s0);
  s1 = wave_sum(s1);
  if (lane == 0) {
    sh.ss[slot][0][2 * wave] = s0;
    sh.ss[slot][0][2 * wave + 1] = s1;
  }
}

// inv_rms of token tt from the sums-of-squares partials of slot `slot`.  With
// row sums (RSS) the total sits in ss[slot][0] and the other partials are
// zero: reading it alone gives the same bits as adding the zeros.
template <int N, int FD, bool RSS = false>
__device__ __forceinline__ float persist_inv_rms(const PersistShared<N, FD>& sh, int slot, int tt,
                                                 float nc, float eps) {
  float sq = 0.f;
  if constexpr (RSS) {
    sq = sh.ss[slot][0][tt];
  } else {
#pragma unroll
    for (int w = 0; w < kPersistWaves; ++w) sq += sh.ss[slot][w][tt];
  }
  return 1.0f / sqrtf(sq / nc + eps);
}

// ---- phase 1: projection partials (MFMA) of x_norm -> LDS.  The A operand is
// the row's x_norm = bf16(x * inv_rms), rounded as the reference's torch op
// rounds it (model/mhc_fused.py:845: (x.float() * inv_rms).to(x.dtype)), so
// the projection sums the same bf16 products the reference's GEMM sums.
template <int N, int MODE, int KB, bool NORM, bool RSS = false, typename Issue = NoIssue>
__device__ __forceinline__ void persist_project(
    const PreArgs& a, PersistShared<N, PersistPlan<N, MODE, KB>::FD>& sh, const U32x4 (&xr)[KB][N],
    const bf16x8_t (&wreg)[KB][N][PersistPlan<N, MODE, KB, NORM>::WR], const unsigned char* lds_w,
    int slot, int lane, int wave, const Issue& issue = Issue()) {
  using P = PersistPlan<N, MODE, KB, NORM>;
  constexpr int FD = P::FD;
  constexpr int NT = P::NT;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int NCB = (a.C + kCBlock - 1) / kCBlock;
  const float inv = persist_inv_rms<N, FD, RSS>(sh, slot, r, (float)(N * a.C), a.rms_eps);

  f32x4_t acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Column blocks past C hold zeros in x and in every phi copy (registers, LDS,
  // and the bounded L2 reads below), so every block runs unconditionally: no
  // branch splits the waits on the x buffers.
  const auto wr = make_rsrc(a.phi_packed, (uint32_t)(N * NCB * NT) * 64u * 16u);
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int cb = wave + kPersistWaves * q;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const bf16x8_t av = __builtin_bit_cast(bf16x8_t, x_norm_chunk(xr[q][i], inv));
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
          const uint32_t off =
              cb < NCB ? (uint32_t)(((i * NCB + cb) * NT + nt) * 64 + lane) * 16u : kBufOob;
          bv = __builtin_bit_cast(bf16x8_t, buf_load16(wr, off));
        }
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[nt], 0, 0, 0);
      }
    }
    issue.at(q);
  }
  // MFMA 16x16 result layout: lane l holds D[4*(l/16) + j][l % 16], j = 0..3.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    if (nt * 16 + r < FD)
#pragma unroll
      for (int j = 0; j < 4; ++j) sh.acc[slot][wave][4 * g + j][nt * 16 + r] = acc[nt][j];
}

// ---- gates ---------------------------------------------------------------
// The reduced projection m = sum_w partial of feature f of token tt (of x_norm,
// so already normalised), from partials slot `slot`.
template <int N, int FD>
__device__ __forceinline__ float persist_mix(const PersistShared<N, FD>& sh, int slot, int tt, int f) {
  float sum = 0.f;
#pragma unroll
  for (int w = 0; w < kPersistWaves; ++w) sum += sh.acc[slot][w][tt][f];
  return sum;
}

// h_pre of (token lane / N, stream lane % N) for every wave (lanes past TM*N
// return 0); wave POST_WAVE also writes h_post, h_pre, inv_rms and the
// pre/post mixes when asked for.
template <int N, int MODE, int KB, bool RSS = false>
__device__ __forceinline__ float persist_pre_post(const PreArgs& a,
                                                  const PersistShared<N, PersistPlan<N, MODE, KB>::FD>& sh,
                                                  int64_t tile, int slot, int lane, int wave) {
  using P = PersistPlan<N, MODE, KB>;
  using GP = GateParams<N>;
  constexpr int FD = P::FD;
  float hp = 0.f;
  if (lane < kTokTile * N) {
    const int tt = lane / N;
    const int i = lane % N;
    const float m = persist_mix(sh, slot, tt, i);
    hp = gate_pre(m, sh.prm[0], sh.prm[GP::kBiasPre + i], a.pre_eps, kBF16);
    if (wave == P::POST_WAVE) {
      const int64_t tk = tile * kTokTile + tt;
      const bool ok = tk < a.M;
      if (ok) {
        if (a.h_pre) st_any(a.h_pre, tk * N + i, kBF16, hp);
        if (a.inv_rms && i == 0)
          a.inv_rms[tk] = persist_inv_rms<N, FD, RSS>(sh, slot, tt, (float)(N * a.C), a.rms_eps);
        if (a.mixes_raw) a.mixes_raw[tk * FD + i] = m;
      }
      if constexpr (MODE != kHead) {
        const float mp = persist_mix(sh, slot, tt, N + i);
        const float hq = gate_post(mp, sh.prm[1], sh.prm[GP::kBiasPost + i], a.post_mult, kBF16);
        if (ok) {
          st_any(a.h_post, tk * N + i, kBF16, hq);
          if (a.mixes_raw) a.mixes_raw[tk * FD + N + i] = mp;
        }
      }
    }
  }
  return hp;
}

// h_res logits of the tile, one (token, element) per lane of the gate waves,
// into LDS slot `slot` for the next step's Sinkhorn.
template <int N, int MODE, int KB>
__device__ __forceinline__ void persist_res_gates(const PreArgs& a,
                                                  PersistShared<N, PersistPlan<N, MODE, KB>::FD>& sh,
                                                  int64_t tile, int slot, int idx0) {
  using P = PersistPlan<N, MODE, KB>;
  using GP = GateParams<N>;
  constexpr int FD = P::FD;
  constexpr int G = P::G;
  for (int idx = idx0; idx < kTokTile * G; idx += P::GATE_LANES) {
    const int tt = idx / G;
    const int e = idx % G;
    const float m = persist_mix(sh, slot, tt, 2 * N + e);
    const float h = gate_res(m, sh.prm[2], sh.prm[GP::kBiasRes + e], kBF16);
    sh.hres[slot][idx] = h;
    const int64_t tk = tile * kTokTile + tt;
    if (tk < a.M) {
      if (a.h_res_raw) st_any(a.h_res_raw, tk * G + e, kBF16, h);
      if (a.mixes_raw) a.mixes_raw[tk * FD + 2 * N + e] = m;
    }
  }
}

// ---- phase 2b: Sinkhorn-Knopp of tile `tile` from LDS slot `slot`, one matrix
// element per lane (waves 0..SK_WAVES-1).
template <int N>
__device__ __forceinline__ void persist_sinkhorn(const PreArgs& a, const float* hres, int64_t tile,
                                                 int tid) {
  constexpr int G = N * N;
  constexpr int TM = kTokTile;
  const int64_t t0 = tile * TM;
  const int e = tid;
  float v = e < TM * G ? hres[e] : 0.f;
  v = sinkhorn_lane<N>(v, a.sk_iters, a.sk_eps);
  if (e < TM * G && t0 + e / G < a.M) st_any(a.h_res, t0 * G + e, kBF16, v);
}

// ---- phase 3: pre-aggregate from the held x registers.  With the norm the
// chunks go to the lane's LDS slots and the token's sum of squares (of the
// bf16-rounded values) to this wave's partial, for persist_norm_store.
template <int N, int KB, bool NORM, typename Issue = NoIssue>
__device__ __forceinline__ void persist_preagg(const PreArgs& a, const U32x4 (&xr)[KB][N],
                                               const uint32_t (&hlo)[N], const uint32_t (&hhi)[N],
                                               int64_t tile, int lane, int wave,
                                               PersistNorm<NORM, KB>& nsh, int slot,
                                               const Issue& issue = Issue(),
                                               unsigned char* stage = nullptr) {
  constexpr int TM = kTokTile;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t M = a.M;
  const int C = a.C;
  const int64_t t0 = wave_uniform(tile * TM);
  const int valid = (int)(M - t0 < TM ? M - t0 : TM);
  const auto rsub = make_rsrc(static_cast<uint16_t*>(a.sub_in) + t0 * C, (uint32_t)valid * C * 2u);
  const uint32_t sub_row = (uint32_t)(r * C) * 2u;
  float q2 = 0.f;
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    issue.at(q);
    const int c0 = (wave + kPersistWaves * q) * kCBlock;
    const uint32_t lo = x_lane_off(q, wave, g, C);
    const U32x4 pk = preagg_chunk<N>(xr[q], hlo, hhi);
    if constexpr (NORM) {  // column blocks past C hold zeros
#pragma unroll
      for (int j = 0; j < 4; ++j) q2 = dot2_bf16(pk.v[j], pk.v[j], q2);
      nsh.stash[slot][r * PersistNorm<NORM, KB>::kChunks + (c0 >> 3) + g] = pk;
      continue;
    }
    if (stage) {  // row staging: the tile's rows go out whole at the next step
      // chunk j = 4 wave + g + 32 q of row r; the XOR with r < 16 touches only
      // the low 5 bits, so the three chunks are one base 512 bytes apart
      constexpr int SCH = KB * 32;
      const uint32_t base = (uint32_t)(r * SCH + ((4 * wave + g) ^ r)) * 16u;
      *reinterpret_cast<U32x4*>(stage + base + q * 512) = pk;
      continue;
    }
    // The whole offset travels in the vector offset, the scalar offset stays
    // the literal 0: a 128-bit store reads its data registers after issue, and
    // the compiler only keeps the next VALU write off those registers for
    // stores of that form.  With a register soffset it reused the first data
    // register at once and some lanes stored the new value.
    buf_store16_nt<kNtSc1>(rsub, lo == kBufOob ? kBufOob : sub_row + lo + (uint32_t)c0 * 2u, pk);
  }
  if constexpr (NORM) {
    q2 += __shfl_xor(q2, 16, 64);
    q2 += __shfl_xor(q2, 32, 64);
    if (g == 0) nsh.ss2[slot][wave][r] = q2;
  }
}

// ---- RMSNorm epilogue of tile `tile` (stash and partials slot `slot`), once a
// barrier has made every wave's partial visible: scale the stashed chunks by
// 1 / sqrt(mean_c(s^2) + norm_eps) and the gain, round to bf16, store.
template <int N, int KB>
__device__ __forceinline__ void persist_norm_store(const PreArgs& a, const PersistNorm<true, KB>& nsh,
                                                   int64_t tile, int slot, int lane, int wave) {
  constexpr int TM = kTokTile;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t M = a.M;
  const int C = a.C;
  const int64_t t0 = wave_uniform(tile * TM);
  const int valid = (int)(M - t0 < TM ? M - t0 : TM);
  const auto rsub = make_rsrc(static_cast<uint16_t*>(a.sub_in) + t0 * C, (uint32_t)valid * C * 2u);
  const uint32_t sub_row = (uint32_t)(r * C) * 2u;
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kPersistWaves; ++w) t += nsh.ss2[slot][w][r];
  const float sc = 1.0f / sqrtf(t / (float)C + a.norm_eps);
#pragma unroll
  for (int q = 0; q < KB; ++q) {
    const int c0 = (wave + kPersistWaves * q) * kCBlock;
    const uint32_t lo = x_lane_off(q, wave, g, C);
    const U32x4 pk = nsh.stash[slot][r * PersistNorm<true, KB>::kChunks + (c0 >> 3) + g];
    const float4 w0 = *reinterpret_cast<const float4*>(&nsh.gain[c0 + 8 * g]);
    const float4 w1 = *reinterpret_cast<const float4*>(&nsh.gain[c0 + 8 * g + 4]);
    U32x4 y;
    y.v[0] = pack_bf16x2(bf16lo(pk.v[0]) * sc * w0.x, bf16hi(pk.v[0]) * sc * w0.y);
    y.v[1] = pack_bf16x2(bf16lo(pk.v[1]) * sc * w0.z, bf16hi(pk.v[1]) * sc * w0.w);
    y.v[2] = pack_bf16x2(bf16lo(pk.v[2]) * sc * w1.x, bf16hi(pk.v[2]) * sc * w1.y);
    y.v[3] = pack_bf16x2(bf16lo(pk.v[3]) * sc * w1.z, bf16hi(pk.v[3]) * sc * w1.w);
    // whole offset in the vector offset, scalar offset the literal 0 (see above)
    buf_store16_nt<kNtSc1>(rsub, lo == kBufOob ? kBufOob : sub_row + lo + (uint32_t)c0 * 2u, y);
  }
}

// Row staging: the sublayer input of tile `tile`, staged in LDS by its
// pre-aggregate (chunk j of row r at (r * SCH + (j ^ r)) * 16, the XOR
// spreading the 16 rows of one column over the banks), stored as whole rows:
// wave w takes the two-row span of rows 2w and 2w + 1, lane l its chunks l,
// l + 64, .. (1 KiB per wave instruction), where the pre-aggregate's own
// layout splits every 128-byte line of sub_in between two waves.
template <int KB>
__device__ __forceinline__ void persist_stage_store(const PreArgs& a, const unsigned char* stage,
                                                    int64_t tile, int lane, int wave) {
  constexpr int SCH = KB * 32;
  const int64_t M = a.M;
  const int C = a.C;
  const int64_t t0 = wave_uniform(tile * kTokTile);
  const int valid = (int)(M - t0 < kTokTile ? M - t0 : kTokTile);
  const auto rsub = make_rsrc(static_cast<uint16_t*>(a.sub_in) + t0 * C, (uint32_t)valid * C * 2u);
#pragma unroll
  for (int k = 0; k < KB; ++k) {
    const int qr = lane + 64 * k;        // chunk of the two-row span of rows 2w, 2w + 1
    const int second = qr >= SCH ? 1 : 0;
    const int j = qr - second * SCH;     // chunk of its row
    const int row = 2 * wave + second;   // < 16: row & 15 == row
    const U32x4 v = *reinterpret_cast<const U32x4*>(stage + (row * SCH + (j ^ row)) * 16);
    // whole offset in the vector offset, scalar offset the literal 0 (see persist_preagg)
    buf_store16_nt<kNtSc1>(rsub, (uint32_t)(2 * wave * SCH + qr) * 16u, v);
  }
}

// One tile (sums-of-squares, partials and h_res slot `slot`); the next tile's
// loads go into xn in three batches along the way.
template <int N, int MODE, int KB, bool NORM>
__device__ __forceinline__ void persist_step(
    const PreArgs& a, PersistShared<N, PersistPlan<N, MODE, KB>::FD>& sh, PersistNorm<NORM, KB>& nsh,
    const U32x4 (&xr)[KB][N], U32x4 (&xn)[KB][N],
    const bf16x8_t (&wreg)[KB][N][PersistPlan<N, MODE, KB, NORM>::WR], const unsigned char* lds_w,
    int64_t tile, int64_t prev, int64_t ntiles, int slot, int tid, int lane, int wave) {
  using P = PersistPlan<N, MODE, KB, NORM>;
  const int r = lane & 15;
  const int g = lane >> 4;
  const auto rn = x_tile_rsrc(static_cast<const uint16_t*>(a.x), tile + gridDim.x, ntiles, a.M,
                              N * a.C);
  persist_load_part<N, KB, 0, P::B1>(xn, rn, a.C, wave, r, g);
  persist_sumsq(sh, xr, slot, lane, wave);
  __syncthreads();  // sums of squares visible
  persist_load_part<N, KB, P::B1, P::B2>(xn, rn, a.C, wave, r, g);
  persist_project<N, MODE, KB, NORM>(a, sh, xr, wreg, lds_w, slot, lane, wave);
  __syncthreads();  // partials visible
  if constexpr (MODE == kFull) {
    if (wave < P::SK_WAVES && prev >= 0 && a.h_res)
      persist_sinkhorn<N>(a, sh.hres[slot ^ 1], prev, tid);
  }
  const float hp = persist_pre_post<N, MODE, KB>(a, sh, tile, slot, lane, wave);
  if constexpr (MODE == kFull) {
    if (wave >= P::SK_WAVES) persist_res_gates<N, MODE, KB>(a, sh, tile, slot, tid - P::SK_WAVES * 64);
  }
  uint32_t hlo[N];
  uint32_t hhi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {  // h_pre of this lane's token r, stream i
    const float h = __shfl(hp, r * N + i, 64);
    hlo[i] = pack_lo(h);
    hhi[i] = pack_hi(h);
  }
  persist_preagg<N, KB, NORM>(a, xr, hlo, hhi, tile, lane, wave, nsh, slot);
  persist_load_part<N, KB, P::B2, KB>(xn, rn, a.C, wave, r, g);
  // The previous tile's normed stores, here where this tile's x registers are
  // free (its partials became visible at this step's barrier).
  if constexpr (NORM) {
    if (prev >= 0) persist_norm_store<N, KB>(a, nsh, prev, slot ^ 1, lane, wave);
  }
}

// One tile with row staging: xn holds the tile in row layout (its loads were
// issued during the previous step); it goes to LDS, each wave sums the squares
// of its two rows from xn, xn takes the next tile's loads in three parts along
// the step (at its start, spread through the projection, spread through the
// pre-aggregate), and the operand registers xr are read back from LDS.  The
// first barrier orders the LDS writes (tile and row sums) before the reads;
// the previous step's partials barrier orders this step's writes after every
// wave's previous reads.  (The row sums replace the operand-layout partial
// sums and the barrier after them: C2 pre 31.4 -> 29.9 us on MI355X.)  (Overlapping two tiles' loads, with the LDS tile
// taking the next tile's first batch once read, measured slower: the extra
// loads in flight stall the issuing waves.)
template <int N, int MODE, int KB>
__device__ __forceinline__ void persist_step_row(
    const PreArgs& a, PersistShared<N, PersistPlan<N, MODE, KB>::FD>& sh, PersistNorm<false, KB>& nsh,
    unsigned char* xl, unsigned char* stage, U32x4 (&xr)[KB][N], U32x4 (&xn)[KB][N],
    const bf16x8_t (&wreg)[KB][N][PersistPlan<N, MODE, KB>::WR], const unsigned char* lds_w,
    int64_t tile, int64_t prev, int64_t ntiles, int slot, int tid, int lane, int wave, bool last) {
  using P = PersistPlan<N, MODE, KB>;
  using RW = PersistRow<N, MODE, KB>;
  const int r = lane & 15;
  const auto rn = x_tile_rsrc(static_cast<const uint16_t*>(a.x), tile + gridDim.x, ntiles, a.M,
                              N * a.C);
  persist_row_to_lds<N, MODE, KB, 0, RW::PW>(xl, xn, wave, lane);
  persist_row_sumsq<N, MODE, KB>(sh, xn, slot, wave, lane);
  if constexpr (!RW::STAGE) persist_load_row<N, MODE, KB, 0, RW::R1>(xn, rn, wave, lane);
  __syncthreads();  // the tile in LDS, its row sums of squares and the previous sub_in visible
  if constexpr (RW::STAGE) {
    // The previous tile's sublayer input goes out while neither the operand
    // registers nor the next tile's loads are live.
    if (prev >= 0) persist_stage_store<KB>(a, stage, prev, lane, wave);
    persist_load_row<N, MODE, KB, 0, RW::R1>(xn, rn, wave, lane);
  }
  persist_lds_to_operands<N, MODE, KB>(xl, xr, wave, lane);
  persist_project<N, MODE, KB, false, true>(a, sh, xr, wreg, lds_w, slot, lane, wave,
                                      RowIssue<N, MODE, KB, RW::R1, RW::R2>{xn, rn, wave, lane});
  __syncthreads();  // partials visible
  if constexpr (MODE == kFull) {
    // In the last step the previous tile's Sinkhorn waits for the end of the
    // loop, where it runs on the gate waves beside the last tile's.
    if (wave < P::SK_WAVES && prev >= 0 && a.h_res && !last)
      persist_sinkhorn<N>(a, sh.hres[slot ^ 1], prev, tid);
  }
  const float hp = persist_pre_post<N, MODE, KB, true>(a, sh, tile, slot, lane, wave);
  uint32_t hlo[N];
  uint32_t hhi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {  // h_pre of this lane's token r, stream i
    const float h = __shfl(hp, r * N + i, 64);
    hlo[i] = pack_lo(h);
    hhi[i] = pack_hi(h);
  }
  persist_preagg<N, KB, false>(a, xr, hlo, hhi, tile, lane, wave, nsh, slot,
                               RowIssue<N, MODE, KB, RW::R2, RW::PW>{xn, rn, wave, lane},
                               RW::STAGE ? stage : nullptr);
  // The h_res logits feed the next step's Sinkhorn only: after the
  // pre-aggregate, whose stores and next-tile loads then go out sooner, they
  // overlap the wait for those loads (C2 pre 29.2 -> 28.9 us).
  if constexpr (MODE == kFull) {
    if (wave >= P::SK_WAVES) persist_res_gates<N, MODE, KB>(a, sh, tile, slot, tid - P::SK_WAVES * 64);
  }
}

// Gate parameter of thread tid (raw bits; converted once the streaming loads
// are out).  Branch-free: threads without a parameter read alpha_pre[0].
struct RawParam {
  uint32_t lo, hi;
  bool used;
};

template <int N, int MODE>
__device__ __forceinline__ RawParam load_gate_param(const PreArgs& a, int tid) {
  using GP = GateParams<N>;
  int which = 5;
  int idx = tid - GP::kBiasRes;
  if (tid < GP::kBiasRes) { which = 4; idx = tid - GP::kBiasPost; }
  if (tid < GP::kBiasPost) { which = 3; idx = tid - GP::kBiasPre; }
  if (tid < 3) { which = tid; idx = 0; }
  const bool used = tid < GP::kCount &&
                    (which == 0 || which == 3 ||
                     (MODE != kHead && (which == 1 || which == 4)) ||
                     (MODE == kFull && (which == 2 || which == 5)));
  const void* p = a.alpha[0];
  p = which == 1 ? a.alpha[1] : p;
  p = which == 2 ? a.alpha[2] : p;
  p = which == 3 ? a.bias[0] : p;
  p = which == 4 ? a.bias[1] : p;
  p = which == 5 ? a.bias[2] : p;
  p = used ? p : a.alpha[0];
  idx = used ? idx : 0;
  const int es = a.param_dtype == kF32 ? 4 : 2;
  const unsigned char* b = static_cast<const unsigned char*>(p) + (int64_t)idx * es;
  RawParam rp;
  rp.lo = *reinterpret_cast<const uint16_t*>(b);
  rp.hi = *reinterpret_cast<const uint16_t*>(b + (es == 4 ? 2 : 0));
  rp.used = used;
  return rp;
}

__device__ __forceinline__ float convert_param(const RawParam& rp, int dt) {
  const float f32 = __uint_as_float(rp.lo | (rp.hi << 16));
  const float bf = __uint_as_float(rp.lo << 16);
  const float f16 = f16_bits_to_f32((uint16_t)rp.lo);
  const float v = dt == kF32 ? f32 : (dt == kBF16 ? bf : f16);
  return rp.used ? v : 0.f;
}

template <int N, int MODE, int KB, bool NORM, bool ROW = false>
__global__ __launch_bounds__(kPersistWaves * 64) void pre_persist_kernel(PreArgs a, int64_t ntiles) {
  using P = PersistPlan<N, MODE, KB, NORM>;
  using RW = PersistRow<N, MODE, KB>;
  static_assert(P::SHARED + 256 + (P::NLDS > 0 ? P::LDS_W : 0) <= kLdsBytes, "LDS budget");
  static_assert(!ROW || (RW::OK && !NORM), "row staging: C == 256 * KB, phi in registers, no norm");
  __shared__ PersistShared<N, P::FD> sh;
  __shared__ PersistNorm<NORM, KB> nsh;
  __shared__ __attribute__((aligned(16))) unsigned char lds_w[P::LDS_W];
  __shared__ __attribute__((aligned(16))) unsigned char xl[ROW ? RW::BYTES : 16];
  __shared__ __attribute__((aligned(16))) unsigned char sub_stage[ROW && RW::STAGE ? RW::SUBB : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int r = lane & 15;
  const int g = lane >> 4;
  const int C = a.C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(a.x);
  const int64_t step = gridDim.x;
  int64_t tile = blockIdx.x;

  // Issue order: gate parameters, register phi tiles, the first x tile (when
  // it fits beside the LDS phi staging), LDS phi tiles, the first x tile
  // otherwise.  The LDS writes wait only for phi.  Padding lanes of a compact
  // phi tile write into the (not yet used) partials area.  The second tile's
  // loads go out during the first step.
  const RawParam rp = load_gate_param<N, MODE>(a, tid);
  // norm gain words of columns tid and tid + 512, converted where they are
  // stored to LDS (ld_any's per-dtype branch made the prologue's loads wait)
  uint32_t gain_w[2] = {0u, 0u};
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * kPersistWaves * 64;
      gain_w[h] = ld_word(a.norm_w, C, c < C ? c : 0, a.norm_dtype);
    }
  }

  const uint32_t wbytes = (uint32_t)(N * NCB * P::NT) * 64u * 16u;
  const auto wr = make_rsrc(a.phi_packed, wbytes);
  // Lanes of the last 16-column tile past FD hold zero operands (the packed
  // image stores zeros there): they read nothing (out-of-range offset), which
  // takes a quarter of the start-up phi traffic away at n = 4 (FD = 24).
  auto phi_off = [&](int nt, int q, int i) -> uint32_t {
    const int cb = wave + kPersistWaves * q;
    const bool pad = nt == P::NT - 1 && r >= P::LAST_COLS;
    return cb < NCB && !pad ? (uint32_t)(((i * NCB + cb) * P::NT + nt) * 64 + lane) * 16u : kBufOob;
  };
  bf16x8_t wreg[KB][N][P::WR];
#pragma unroll
  for (int nt = 0; nt < P::NREG; ++nt)
#pragma unroll
    for (int q = 0; q < KB; ++q)
#pragma unroll
      for (int i = 0; i < N; ++i)
        wreg[q][i][nt] = __builtin_bit_cast(bf16x8_t, buf_load16(wr, phi_off(nt, q, i)));

  U32x4 xa[KB][N];
  U32x4 xb[KB][N];
  const auto r0 = x_tile_rsrc(x, tile, ntiles, a.M, N * C);
  if constexpr (ROW) persist_load_row<N, MODE, KB, 0, RW::PW>(xa, r0, wave, lane);
  else if constexpr (P::X_EARLY) persist_load_part<N, KB, 0, KB>(xa, r0, C, wave, r, g);
  constexpr int NST = P::NLDS > 0 ? P::NLDS : 1;
  U32x4 st[NST][KB][N];  // LDS phi tiles, staged
#pragma unroll
  for (int t = 0; t < P::NLDS; ++t)
#pragma unroll
    for (int q = 0; q < KB; ++q)
#pragma unroll
      for (int i = 0; i < N; ++i) st[t][q][i] = buf_load16(wr, phi_off(P::NREG + t, q, i));
#pragma unroll
  for (int t = 0; t < P::NLDS; ++t) {
    const int nt = P::NREG + t;
    const int cols = P::cols(nt);
#pragma unroll
    for (int q = 0; q < KB; ++q)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        unsigned char* dst = r < cols ? lds_w + P::lds_base(nt) +
                                            ((((wave * KB + q) * N + i) * 4 + g) * cols + r) * 16
                                      : reinterpret_cast<unsigned char*>(&sh.acc[0][0][0]) + lane * 16;
        *reinterpret_cast<U32x4*>(dst) = st[t][q][i];
      }
  }
  if constexpr (!P::X_EARLY && !ROW) persist_load_part<N, KB, 0, KB>(xa, r0, C, wave, r, g);

  if (tid == 0) sh.zero = U32x4{{0u, 0u, 0u, 0u}};
  if constexpr (ROW) {  // the row sums live in ss[slot][0]; the other partials stay zero
    constexpr int kRest = 2 * (kPersistWaves - 1) * kTokTile;
    if (tid < kRest)
      sh.ss[tid / ((kPersistWaves - 1) * kTokTile)][1 + (tid / kTokTile) % (kPersistWaves - 1)][tid % kTokTile] = 0.f;
  }
  if (tid < GateParams<N>::kCount) sh.prm[tid] = convert_param(rp, a.param_dtype);
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * kPersistWaves * 64;
      nsh.gain[c] = c < C ? word_elem(gain_w[h], c, a.norm_dtype) : 0.f;
    }
  }
  __syncthreads();  // gate parameters, zero block and phi tiles visible

  // Pairs of steps (xa computes while xb loads, then the reverse), then the
  // leftover step.  The loop body has no exit between its steps: an exit
  // there leaves the compiler a path into the loop header on which the
  // prefetch order differs, and the header then waits for every load in
  // flight.
  const int64_t my_tiles = (ntiles - blockIdx.x + step - 1) / step;
  int64_t prev = -1;
  int64_t pprev = -1;  // the tile before prev (row staging: its Sinkhorn runs after the loop)
  int slot = 0;
  int64_t k = 0;
  if constexpr (ROW) {  // fixed roles: xa in flight (row layout), xb the operands
    for (; k < my_tiles; ++k) {
      persist_step_row<N, MODE, KB>(a, sh, nsh, xl, sub_stage, xb, xa, wreg, lds_w, tile, prev, ntiles,
                                    slot, tid, lane, wave, k + 1 == my_tiles);
      pprev = prev;
      prev = tile;
      slot ^= 1;
      tile += step;
    }
  }
  for (; !ROW && k + 2 <= my_tiles; k += 2) {  // uniform across the workgroup
    persist_step<N, MODE, KB, NORM>(a, sh, nsh, xa, xb, wreg, lds_w, tile, prev, ntiles, slot, tid, lane, wave);
    prev = tile;
    slot ^= 1;
    tile += step;
    persist_step<N, MODE, KB, NORM>(a, sh, nsh, xb, xa, wreg, lds_w, tile, prev, ntiles, slot, tid, lane, wave);
    prev = tile;
    slot ^= 1;
    tile += step;
  }
  if (!ROW && k < my_tiles) {
    persist_step<N, MODE, KB, NORM>(a, sh, nsh, xa, xb, wreg, lds_w, tile, prev, ntiles, slot, tid, lane, wave);
    prev = tile;
    slot ^= 1;
  }
  // The last tile's Sinkhorn, once every gate wave has written its logits,
  // its normed stores, once every wave has written its partial, and (row
  // staging) its staged sublayer input.
  if constexpr (MODE == kFull || NORM || (ROW && RW::STAGE)) __syncthreads();
  if constexpr (ROW && RW::STAGE) persist_stage_store<KB>(a, sub_stage, prev, lane, wave);
  if constexpr (NORM) persist_norm_store<N, KB>(a, nsh, prev, slot ^ 1, lane, wave);
  if constexpr (MODE == kFull) {
    if (wave < P::SK_WAVES && a.h_res) persist_sinkhorn<N>(a, sh.hres[slot ^ 1], prev, tid);
    // Row staging: the tile before the last, deferred from the last step, on
    // the gate waves (each SIMD then interleaves two independent Sinkhorn
    // chains); its logits sit in the other slot, untouched since its step.
    if constexpr (ROW) {
      if (wave >= P::SK_WAVES && wave < 2 * P::SK_WAVES && pprev >= 0 && a.h_res)
        persist_sinkhorn<N>(a, sh.hres[slot], pprev, tid - P::SK_WAVES * 64);
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
  if constexpr (PersistRow<N, MODE, KB>::OK) {
    if (!a.norm_w && a.C == 256 * KB && pre_row_staging()) {
      hipLaunchKernelGGL((pre_persist_kernel<N, MODE, KB, false, true>), dim3((unsigned)grid),
                         dim3(kPersistWaves * 64), 0, s, a, ntiles);
      return hipGetLastError();
    }
  }
  if (a.norm_w)
    hipLaunchKernelGGL((pre_persist_kernel<N, MODE, KB, true>), dim3((unsigned)grid),
                       dim3(kPersistWaves * 64), 0, s, a, ntiles);
  else
    hipLaunchKernelGGL((pre_persist_kernel<N, MODE, KB, false>), dim3((unsigned)grid),
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
