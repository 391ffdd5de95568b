// Pre phase for small batches: one workgroup per token (bf16 streams, packed
// phi, n <= 2, C <= 1024, C % 8 == 0).
//
// At decode sizes (tens of tokens) the persistent kernel runs one 16-token
// tile per workgroup on a handful of CUs, each of which first pulls all of phi
// into registers: the launch is a chain of latencies on few CUs.  Here every
// token gets a workgroup of its own and every step is short.  Each workgroup
// still reads all of phi from L2 (n*C*FD bf16), so this pays only while phi is
// small: measured on MI355X at C = 768, n = 2 (phi 24 KB) it beats the
// persistent kernel up to ~512 tokens (5.0 vs 6.0 us at 64); at n = 4 (phi
// 147 KB) the per-workgroup phi reads make it slower at every size (10.2 vs
// 9.2 us at 64), so n = 4 stays on the persistent kernel.
//   * thread t owns columns 8t .. 8t+7 of every stream: one 16-byte x chunk
//     per stream, read once, held in registers until the pre-aggregate;
//   * the sum of squares and the FD projection partials are bf16 dot2 over
//     those chunks; the phi operand comes from the packed MFMA image of phi
//     (16 bytes = 8 consecutive rows k of one output column f), read from L2;
//   * wave butterflies and one LDS pass reduce the FD + 1 partials; thread f
//     then forms feature f's gate (parameters loaded at kernel start);
//   * the pre-aggregate is thread-local (all n streams of the thread's
//     columns), with the optional RMSNorm over C after one more reduction;
//   * the Sinkhorn runs one matrix element per lane on the last wave, after
//     that wave's share of the pre-aggregate.
// Arithmetic and rounding are those of the persistent kernel: ss and the
// projection accumulate in fp32 over bf16 products, mixes = acc * inv_rms,
// gates rounded as the reference's torch ops round (model/mhc_fused.py:533-559),
// Sinkhorn per model/mhc_fused.py:47-56, pre-aggregate per :556-557.
#include "mhc_pre_persist.hpp"

namespace mhc {

namespace {
// Measured crossover with the persistent kernel (n = 2, C = 768 on MI355X).
int64_t g_token_max_m = 512;
}  // namespace

int64_t pre_token_max_m() { return g_token_max_m; }
void set_pre_token_max_m(int64_t m) { g_token_max_m = m; }

namespace {
bool g_row_staging = true;
}  // namespace

bool pre_row_staging() { return g_row_staging; }
void set_pre_row_staging(bool on) { g_row_staging = on; }

constexpr int kTokThreads = 128;  // 128 column groups of 8: C <= 1024

template <int N, int MODE>
__global__ __launch_bounds__(kTokThreads) void pre_token_kernel(PreArgs a) {
  using S = PreShape<N, MODE>;
  constexpr int FD = S::FD;
  constexpr int NT = S::NT;
  constexpr int G = N * N;
  constexpr int NW = kTokThreads / 64;
  constexpr int R = FD + 1;  // FD projection partials, then the sum of squares
  __shared__ float s_red[NW][R];
  __shared__ float s_hpre[N];
  __shared__ float s_hres[G];
  __shared__ float s_nrm[NW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t tok = blockIdx.x;
  const int C = a.C;
  const int NC = N * C;
  const int NCB = (C + kCBlock - 1) / kCBlock;
  const bool own = tid < (C >> 3);

  // Gate parameters of feature f = tid, issued before the streaming loads.
  const int pdt = a.param_dtype;
  float g_alpha = 0.f;
  float g_bias = 0.f;
  if (tid < FD) {
    const int seg = tid < N ? 0 : (tid < 2 * N ? 1 : 2);
    g_alpha = ld_any(a.alpha[seg], 0, pdt);
    g_bias = ld_any(a.bias[seg], tid - seg * N, pdt);
  }

  // x: one 16-byte chunk per stream (zeros for threads past C).
  const auto rx = make_rsrc(static_cast<const uint16_t*>(a.x) + tok * NC, (uint32_t)NC * 2u);
  const uint32_t xo = own ? (uint32_t)tid * 16u : kBufOob;
  U32x4 xv[N];
#pragma unroll
  for (int i = 0; i < N; ++i)
    xv[i] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xo, i * C * 2, 0));

  // Norm gain of the thread's columns.
  float gw[8];
  const bool norm = a.norm_w != nullptr;
#pragma unroll
  for (int s = 0; s < 8; ++s) gw[s] = norm && own ? ld_any(a.norm_w, tid * 8 + s, a.norm_dtype) : 0.f;

  // Projection partials against the packed phi (lane image of column block
  // cb = tid / 4, 8-row group g = tid % 4), and the sum of squares.
  float acc[R];
#pragma unroll
  for (int f = 0; f < R; ++f) acc[f] = 0.f;
  const auto rw = make_rsrc(a.phi_packed, (uint32_t)(N * NCB * NT) * 64u * 16u);
  const int cb = tid >> 2;
  const int g = tid & 3;
#pragma unroll
  for (int i = 0; i < N; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[FD] = dot2_bf16(xv[i].v[j], xv[i].v[j], acc[FD]);
#pragma unroll
    for (int f = 0; f < FD; ++f) {
      const uint32_t off =
          own ? (uint32_t)((((i * NCB + cb) * NT + (f >> 4)) * 64) + g * 16 + (f & 15)) * 16u : kBufOob;
      const U32x4 w = buf_load16(rw, off);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[f] = dot2_bf16(xv[i].v[j], w.v[j], acc[f]);
    }
  }
#pragma unroll
  for (int f = 0; f < R; ++f) {
    const float v = wave_sum(acc[f]);
    if (lane == 0) s_red[wave][f] = v;
  }
  __syncthreads();

  // inv_rms and the gates, feature f = tid.
  float ssq = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) ssq += s_red[w][FD];
  const float inv = 1.0f / sqrtf(ssq / (float)NC + a.rms_eps);
  if (tid == 0 && a.inv_rms) a.inv_rms[tok] = inv;
  if (tid < FD) {
    float m = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) m += s_red[w][tid];
    m *= inv;
    if (a.mixes_raw) a.mixes_raw[tok * FD + tid] = m;
    if (tid < N) {
      const float h = gate_pre(m, g_alpha, g_bias, a.pre_eps, kBF16);
      s_hpre[tid] = h;
      if (a.h_pre) st_any(a.h_pre, tok * N + tid, kBF16, h);
    } else if (tid < 2 * N) {
      st_any(a.h_post, tok * N + (tid - N), kBF16, gate_post(m, g_alpha, g_bias, a.post_mult, kBF16));
    } else {
      const int e = tid - 2 * N;
      const float h = gate_res(m, g_alpha, g_bias, kBF16);
      s_hres[e] = h;
      if (a.h_res_raw) st_any(a.h_res_raw, tok * G + e, kBF16, h);
    }
  }
  __syncthreads();

  // Pre-aggregate (MHCHead: the weighted reduce), optionally RMS-normed over C.
  uint32_t hlo[N];
  uint32_t hhi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    hlo[i] = pack_lo(s_hpre[i]);
    hhi[i] = pack_hi(s_hpre[i]);
  }
  U32x4 pk = preagg_chunk<N>(xv, hlo, hhi);
  if (norm) {  // uniform
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) q = dot2_bf16(pk.v[j], pk.v[j], q);
    q = wave_sum(q);
    if (lane == 0) s_nrm[wave] = q;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += s_nrm[w];
    const float r = 1.0f / sqrtf(t / (float)C + a.norm_eps);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      pk.v[j] = pack_bf16x2(bf16lo(pk.v[j]) * r * gw[2 * j], bf16hi(pk.v[j]) * r * gw[2 * j + 1]);
  }
  const auto rs = make_rsrc(static_cast<uint16_t*>(a.sub_in) + tok * C, (uint32_t)C * 2u);
  buf_store16(rs, xo, pk);

  if constexpr (MODE == kFull) {
    if (wave == NW - 1 && a.h_res) {
      float v = lane < G ? s_hres[lane] : 0.f;
      v = sinkhorn_lane<N>(v, a.sk_iters, a.sk_eps);
      if (lane < G) st_any(a.h_res, tok * G + lane, kBF16, v);
    }
  }
}

bool pre_token_supported(const PreArgs& a) {
  if (a.x_dtype != kBF16 || !a.phi_packed) return false;
  if (!(a.n == 1 || a.n == 2)) return false;
  if (!(a.mode == kFull || a.mode == kNoHres || (a.mode == kHead && a.n > 1))) return false;
  return a.C % 8 == 0 && a.C / 8 <= kTokThreads;
}

template <int N, int MODE>
hipError_t launch_pre_token_inst(const PreArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((pre_token_kernel<N, MODE>), dim3((unsigned)a.M), dim3(kTokThreads), 0, s, a);
  return hipGetLastError();
}

template <int N>
hipError_t launch_pre_token_n(const PreArgs& a, hipStream_t s) {
  switch (a.mode) {
    case kFull: return launch_pre_token_inst<N, kFull>(a, s);
    case kNoHres: return launch_pre_token_inst<N, kNoHres>(a, s);
    case kHead:
      if constexpr (N > 1) return launch_pre_token_inst<N, kHead>(a, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pre_token(const PreArgs& a, hipStream_t s) {
  switch (a.n) {
    case 1: return launch_pre_token_n<1>(a, s);
    case 2: return launch_pre_token_n<2>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mhc
