// Backward of the pre phase, its weight gradients, and Sinkhorn-Knopp.
//
// Pre phase, per token (model/mhc_fused.py:271-413; no-H_res
// model/mhc_fused_no_hres.py:150-281; MHCHead model/mhc_common.py:200-295),
// recomputed in fp32 from the saved inv_rms and mixes_raw:
//   gh[i]      = g_h_pre[i] + sum_c g_sub[c] * x[i, c]
//   g_raw      = [gh * s_pre (1 - s_pre),  g_h_post * s_post (1 - s_post) * post_mult,  g_h_res_raw]
//                s_* = sigmoid(alpha_* * mixes + bias_*)
//   gxn[k]     = sum_f alpha_seg(f) g_raw[f] * phi[k, f]
//   g_x[k]     = inv * (gxn[k] - xn[k] * mean_k(xn * gxn)) + (s_pre[i(k)] + pre_eps) * g_sub[c(k)]
//   with mean_k(xn * gxn) = sum_f alpha_seg(f) g_raw[f] mixes_raw[f] / (n*C), since
//   mixes_raw[f] = sum_k xn[k] phi[k, f] (the saved fp32 projection).
// The per-token g_raw (fp32) feeds the weight gradients (model/mhc_fused.py:696-711):
//   grad_phi = alpha_seg * (x * inv)^T @ g_raw,  grad_bias = sum_t g_raw,
//   grad_alpha = sum_t sum_seg g_raw * mixes.
// Sinkhorn backward: the reference recomputes the forward under autograd
// (model/mhc_fused.py:131-137); here the forward iterates are recomputed into
// registers (or LDS for long schedules) and the chain rule runs back through them.
#include "mhc_internal.hpp"

namespace mhc {

namespace {

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is reused by consecutive calls
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

constexpr int kMaxFD = 2 * 16 + 16 * 16;

}  // namespace

// ------------------------------------------------ pre phase, any dtype / shape
// One 256-thread workgroup per token.
__global__ __launch_bounds__(256) void pre_bwd_generic_kernel(PreBwdArgs a) {
  __shared__ float red[4];
  __shared__ float s_gm[kMaxFD];
  __shared__ float s_h[16];
  __shared__ float s_gh[16];
  const int64_t tok = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = a.n;
  const int C = a.C;
  const int64_t NC = (int64_t)n * C;
  const int64_t xb = tok * NC;
  const int xdt = a.x_dtype;
  const int gdt = a.grad_dtype;
  const float inv = a.inv_rms[tok];

  if (a.mode == kRms) {  // y = x * inv_rms: g_x = inv * (g - xn * mean(xn * g))
    float part = 0.f;
    for (int64_t k = tid; k < NC; k += 256)
      part = fmaf(ld_any(a.x, xb + k, xdt) * inv, ld_any(a.g_sub, xb + k, gdt), part);
    const float mean = block_sum(part, red) / (float)NC;
    for (int64_t k = tid; k < NC; k += 256) {
      const float xn = ld_any(a.x, xb + k, xdt) * inv;
      st_any(a.g_x, xb + k, xdt, inv * (ld_any(a.g_sub, xb + k, gdt) - xn * mean));
    }
    return;
  }

  const int FD = mode_fd(a.mode, n);
  for (int i = 0; i < n; ++i) {  // uniform
    float part = 0.f;
    if (a.g_sub)
      for (int c = tid; c < C; c += 256)
        part = fmaf(ld_any(a.g_sub, tok * C + c, gdt), ld_any(a.x, xb + (int64_t)i * C + c, xdt), part);
    const float t = block_sum(part, red);
    if (tid == 0) s_gh[i] = t + (a.g_hpre ? ld_any(a.g_hpre, tok * n + i, gdt) : 0.f);
  }
  __syncthreads();
  for (int f = tid; f < FD; f += 256) {  // FD = 288 at n = 16
    const float m = a.mixes[tok * FD + f];
    const int pdt = a.param_dtype;
    float graw, alpha;
    if (f < n) {
      alpha = ld_any(a.alpha[0], 0, pdt);
      const float sg = sigmoid_f(fmaf(alpha, m, ld_any(a.bias[0], f, pdt)));
      graw = s_gh[f] * sg * (1.0f - sg);
      s_h[f] = sg + a.pre_eps;
    } else if (f < 2 * n) {
      alpha = ld_any(a.alpha[1], 0, pdt);
      const float sg = sigmoid_f(fmaf(alpha, m, ld_any(a.bias[1], f - n, pdt)));
      const float gp = a.g_hpost ? ld_any(a.g_hpost, tok * n + (f - n), gdt) : 0.f;
      graw = gp * sg * (1.0f - sg) * a.post_mult;
    } else {
      alpha = ld_any(a.alpha[2], 0, pdt);
      graw = a.g_hres ? ld_any(a.g_hres, tok * n * n + (f - 2 * n), gdt) : 0.f;
    }
    if (a.g_raw) a.g_raw[tok * FD + f] = graw;
    s_gm[f] = graw * alpha;
  }
  __syncthreads();
  const int pdt = a.phi_dtype;
  float part = 0.f;
  for (int64_t k = tid; k < NC; k += 256) {
    float gxn = 0.f;
    for (int f = 0; f < FD; ++f) gxn = fmaf(s_gm[f], ld_any(a.phi, k * FD + f, pdt), gxn);
    part = fmaf(ld_any(a.x, xb + k, xdt) * inv, gxn, part);
  }
  const float mean = block_sum(part, red) / (float)NC;
  for (int64_t k = tid; k < NC; k += 256) {
    float gxn = 0.f;
    for (int f = 0; f < FD; ++f) gxn = fmaf(s_gm[f], ld_any(a.phi, k * FD + f, pdt), gxn);
    const int i = (int)(k / C);
    const int c = (int)(k - (int64_t)i * C);
    const float xn = ld_any(a.x, xb + k, xdt) * inv;
    const float gs = a.g_sub ? ld_any(a.g_sub, tok * C + c, gdt) : 0.f;
    st_any(a.g_x, xb + k, xdt, inv * (gxn - xn * mean) + s_h[i] * gs);
  }
}

// ------------------------------------------------- pre phase, bf16 on MFMA
// One workgroup of NW waves per 16-token tile.  The tile's n*C row is cut into
// chunks of 32 columns of one stream (chunk k = stream k / NCB, column block
// k % NCB); wave w owns chunks w, w + NW, ...  A lane (r, g) holds token r,
// columns 8g .. 8g + 7 of each of its chunks (16 bytes of x), the layout of
// the forward kernels.
//   A: phi rows.  A-row j of the chunk's k-tile h (h = 0, 1) is column
//      8*(j/4) + 4h + j%4 of the chunk, so the D tile's lane (token c, g),
//      rows 4g .. 4g+3, covers columns 8g + 4h .. 8g + 4h + 3: the two tiles
//      give the 8 columns the lane holds of x.
//   B: (alpha * g_raw)[token][f] for 32 features per K-step, split into bf16
//      hi + lo so the product keeps ~16 mantissa bits (phi is bf16-exact).
// The gh reductions over a token's columns go through the 4 lanes of a token
// (lane xor 16, 32), then per chunk through LDS, summed there in a fixed
// order (deterministic).  mean(xn * gxn) needs no pass over x: it equals
// sum_f gm[f] mixes_raw[f] / NC (gm = alpha * g_raw), formed from LDS with the
// B operands.  So gxn is computed once, straight into g_x, with phi's A
// operands read from L2 as they are used.  That leaves ~90 VGPRs a lane at
// n = 4 (amdgpu_waves_per_eu(4): two 8-wave workgroups per CU), so one
// workgroup's loads overlap the other's gates and MFMAs.
// Eight consecutive elements of a bf16 (one 16-byte load) or fp32 (two)
// tensor, as the MFMA backward kernels hold them.
template <bool F32>
struct Chunk8;
template <>
struct Chunk8<false> {
  U32x4 v;
  __device__ static Chunk8 load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    Chunk8 c;
    c.v = buf_load16(r, off);
    return c;
  }
  // The first K (4 or 2) elements at off, the others zero.
  template <int K>
  __device__ static Chunk8 load_first(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    Chunk8 c;
    c.v = K == 4 ? buf_load8z(r, off) : buf_load4z(r, off);
    return c;
  }
  __device__ static float get(const Chunk8& c, int i) {
    return (i & 1) ? bf16hi(c.v.v[i >> 1]) : bf16lo(c.v.v[i >> 1]);
  }
  // sum_i a[i] * b[i]: exact bf16 products, fp32 sums (v_dot2)
  __device__ static float dot(const Chunk8& a, const Chunk8& b) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = dot2_bf16(a.v.v[e], b.v.v[e], acc);
    return acc;
  }
  __device__ static bf16x8_t hi(const Chunk8& c) { return __builtin_bit_cast(bf16x8_t, c.v); }
  __device__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&x)[8]) {
    U32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.v[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
    buf_store16(r, off, o);
  }
};
template <>
struct Chunk8<true> {
  U32x4 v[2];
  __device__ static Chunk8 load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    Chunk8 c;
    c.v[0] = buf_load16(r, off);
    c.v[1] = buf_load16(r, off == kBufOob ? kBufOob : off + 16u);
    return c;
  }
  template <int K>
  __device__ static Chunk8 load_first(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    Chunk8 c;
    c.v[0] = K == 4 ? buf_load16(r, off) : buf_load8z(r, off);
    c.v[1] = U32x4{{0u, 0u, 0u, 0u}};
    return c;
  }
  __device__ static float get(const Chunk8& c, int i) { return __uint_as_float(c.v[i >> 2].v[i & 3]); }
  __device__ static float dot(const Chunk8& a, const Chunk8& b) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf(get(a, i), get(b, i), acc);
    return acc;
  }
  // bf16(x) and bf16(x - bf16(x)) of the 8 values, as MFMA operands
  __device__ static bf16x8_t hi(const Chunk8& c) {
    U32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.v[e] = pack_bf16x2(get(c, 2 * e), get(c, 2 * e + 1));
    return __builtin_bit_cast(bf16x8_t, o);
  }
  __device__ static bf16x8_t lo(const Chunk8& c) {
    U32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = get(c, 2 * e), a1 = get(c, 2 * e + 1);
      const uint32_t h = pack_bf16x2(a0, a1);
      o.v[e] = pack_bf16x2(a0 - bf16lo(h), a1 - bf16hi(h));
    }
    return __builtin_bit_cast(bf16x8_t, o);
  }
  __device__ static void store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&x)[8]) {
    U32x4 o0, o1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o0.v[e] = __float_as_uint(x[e]);
      o1.v[e] = __float_as_uint(x[4 + e]);
    }
    buf_store16(r, off, o0);
    buf_store16(r, off == kBufOob ? kBufOob : off + 16u, o1);
  }
};

// Row pieces for bf16 x / g_x where C % 64 == 0: C2 pre backward 68.1-69.0 ->
// 64.6-65.4 us, MHCHead 62.9-63.7 -> 60.6-61.1 us, n = 8 (C5) unchanged; with
// the gh sums' g_sub as row pieces too: C2 63.3 -> 60.5 us, C5 97.5 -> 92.4 us,
// MHCHead 59.2 -> 57.2 us (one box).
constexpr bool kPreBwdRowPieces = true;
// Phi operands from contiguous 16-byte pieces of each chunk's phi block,
// regrouped through LDS, instead of 16 phi rows x 64 bytes an instruction:
// C5 pre backward 94.5 -> 76.7 us, C2 61.7 -> 59.7 us (one box); fp32 at
// n = 8, one half of the block at a time: C5 fp32 208.5-210.1 -> 177.6-181.3 us.
constexpr bool kPreBwdPhiBlock = true;
// RS (bf16, or fp32 at n <= 4 where x stays resident; C % 64 == 0; fp32 C2
// 144.4 -> 128.6 us): each wave takes pairs of adjacent chunks (64
// columns of one stream, contiguous in a token's row) and moves the tile's x
// in, g_sub in (for the gh sums) and g_x out as whole 128-byte row pieces,
// regrouped between that layout and the MFMA one through a 2 KiB LDS block of
// its own (no barrier: one wave writes and reads it, in order).  The MFMA
// layout alone covers 16 rows x 64 bytes per load or store, half of each
// 128-byte line.
template <int N, int MODE, int NW, int KJ, bool F32, bool RS = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(F32 ? 2 : 4))) void pre_bwd_mfma_kernel(PreBwdArgs a) {
  using XV = Chunk8<F32>;
  static_assert(!RS || ((!F32 || N <= 4) && KJ % 2 == 0), "row pieces: x resident, whole chunk pairs");
  // The tile's x chunks stay in registers from the gh sums to the g_x stores,
  // except for fp32 at n = 8: 16-wave workgroups hold 128 VGPRs a lane and
  // 12 fp32 chunks alone take 96 of them, so there each chunk is loaded where
  // it is used (for its gh sum, and again with its phi operands for g_x).
  constexpr bool XRES = !(F32 && N >= 8);
  constexpr uint32_t ES = F32 ? 4u : 2u;  // bytes of a stream / gradient / phi element
  constexpr int FD = MODE == kFull ? 2 * N + N * N : (MODE == kNoHres ? 2 * N : N);
  constexpr int KS = (FD + 31) / 32;  // 32-feature K-steps
  constexpr int TM = 16;
  __shared__ float s_gp[NW * KJ][TM];   // per-chunk partials of gh
  __shared__ float s_mx[TM][KS * 32];    // mixes_raw, zero padded
  __shared__ float s_gm[TM][KS * 32];    // alpha * g_raw, zero padded
  __shared__ float s_hp[TM][N];          // h_pre = sigmoid + pre_eps (fp32 recompute)
  // 16-byte pieces: XP per 8 columns, PPR in a chunk pair's row, RPI rows and
  // NRI row-piece loads per pair
  constexpr int XP = F32 ? 2 : 1;
  constexpr int PPR = 8 * XP;
  constexpr int RPI = 64 / PPR;
  constexpr int NRI = TM / RPI;
  __shared__ __attribute__((aligned(16))) U32x4 s_rs[RS ? NW : 1][TM][PPR];  // per-wave regroup block
  // PB: a chunk's phi operands are one contiguous block of phi (its 32 rows x
  // FD features), read with whole 16-byte pieces along the lanes and regrouped
  // into the A layout through a block of LDS per wave.
  // (the shapes whose chunk loop loads a chunk's operand set: KS == 1 or at
  // most 12 chunks a wave)
  // The block is read in half-major order: half h (the A rows of MFMA half h)
  // is the four 4-row groups 8q + 4h .. 8q + 4h + 3, each contiguous in phi.
  // fp32 at n = 8 (x streamed, no row pieces) takes it too, one half in LDS at
  // a time (16 waves x a whole 10 KiB block would not fit).
  constexpr bool PB = FD % 8 == 0 && kPreBwdPhiBlock && (KS == 1 || KJ <= 12) && (RS || (F32 && N >= 8));
  constexpr bool PBH = F32 && N >= 8;      // one half in LDS at a time
  constexpr int GPC = FD * XP / 2;         // 16-byte pieces of a 4-row group
  constexpr int NPH = 4 * GPC;             // of a half
  constexpr int NPBH = (NPH + 63) / 64;    // 64-lane loads of a half
  __shared__ __attribute__((aligned(16))) U32x4 s_pb[PB ? NW : 1][PB ? (PBH ? 1 : 2) * NPH : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int C = a.C;
  const int NC = N * C;
  const int NCB = (C + 31) / 32;
  const int NCH = N * NCB;
  const int64_t t0 = (int64_t)blockIdx.x * TM;
  const int valid = (int)(a.M - t0 < TM ? a.M - t0 : TM);

  const auto rx = make_rsrc(static_cast<const unsigned char*>(a.x) + t0 * NC * ES, (uint32_t)valid * NC * ES);
  const auto rgs = make_rsrc(a.g_sub ? static_cast<const unsigned char*>(a.g_sub) + t0 * C * ES : nullptr,
                             a.g_sub ? (uint32_t)valid * C * ES : 0u);
  const auto rgx = make_rsrc(static_cast<unsigned char*>(a.g_x) + t0 * NC * ES, (uint32_t)valid * NC * ES);

  // chunk j of this wave: stream ci, first column c0; lane column c0 + 8g
  // (RS: chunks 2 (wave + NW j/2) + j % 2, pairs of adjacent ones)
  auto kidx = [&](int j) { return RS ? 2 * (wave + NW * (j >> 1)) + (j & 1) : wave + NW * j; };
  // 16-byte piece e of an 8-column chunk slice (bf16: the one; fp32: two)
  auto piece = [](XV& c, int e) -> U32x4& {
    if constexpr (F32) return c.v[e];
    else { (void)e; return c.v; }
  };
  auto chunk = [&](int j, int& ci, int& c0) {
    const int k = kidx(j);
    ci = k < NCH ? k / NCB : 0;
    c0 = k < NCH ? (k - ci * NCB) * 32 : C;  // C: no columns (loads read zeros)
  };
  auto x_chunk = [&](int j) {
    int ci, c0;
    chunk(j, ci, c0);
    const bool ok = c0 + 8 * g < C;
    return XV::load(rx, ok ? (uint32_t)(r * NC + ci * C + c0 + 8 * g) * ES : kBufOob);
  };
  XV xs[XRES ? KJ : 1];
  if constexpr (XRES) {
    if constexpr (RS) {
      // pair p: row pieces (token RPI i + l / PPR, 16-byte piece l % PPR of the
      // pair's row) into the pair's XV registers, then through LDS into the
      // MFMA layout; piece q of row t sits in slot q ^ (t & 7) (conflict-free
      // both ways)
#pragma unroll
      for (int p = 0; p < KJ / 2; ++p) {
        const int col = 64 * (wave + NW * p);
#pragma unroll
        for (int i = 0; i < NRI; ++i) {
          const int tt = RPI * i + lane / PPR;
          const int pc = lane % PPR;
          piece(xs[2 * p + i / XP], i % XP) =
              buf_load16(rx, col + pc * (16 / (int)ES) < NC ? (uint32_t)(tt * NC + col) * ES + 16u * pc : kBufOob);
        }
      }
#pragma unroll
      for (int p = 0; p < KJ / 2; ++p) {
#pragma unroll
        for (int i = 0; i < NRI; ++i) {
          const int tt = RPI * i + lane / PPR;
          s_rs[wave][tt][(lane % PPR) ^ (tt & 7)] = piece(xs[2 * p + i / XP], i % XP);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < XP; ++e) piece(xs[2 * p + h], e) = s_rs[wave][r][(PPR / 2 * h + XP * g + e) ^ (r & 7)];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      }
    } else {
#pragma unroll
      for (int j = 0; j < KJ; ++j) xs[j] = x_chunk(j);
    }
  }
  const float inv = r < valid ? a.inv_rms[t0 + r] : 0.f;

  // Gate inputs of this thread's (token, feature) items, loaded now so that
  // their latency overlaps the x and g_sub loads instead of following a barrier.
  constexpr int GI = TM * KS * 32;
  constexpr int IPT = (GI + NW * 64 - 1) / (NW * 64);
  const int pdt = a.param_dtype;
  const int gdt = a.grad_dtype;
  float pm[IPT], pg[IPT], pa[IPT], pb[IPT];
#pragma unroll
  for (int q = 0; q < IPT; ++q) {
    const int idx = tid + q * NW * 64;
    const int tt = idx / (KS * 32);
    const int f = idx - tt * (KS * 32);
    pm[q] = pg[q] = pa[q] = pb[q] = 0.f;
    if (idx < GI && f < FD && tt < valid) {
      const int64_t tk = t0 + tt;
      pm[q] = a.mixes[tk * FD + f];
      if (f < N) {
        pg[q] = a.g_hpre ? ld_any(a.g_hpre, tk * N + f, gdt) : 0.f;
        pa[q] = ld_any(a.alpha[0], 0, pdt);
        pb[q] = ld_any(a.bias[0], f, pdt);
      } else if (f < 2 * N) {
        pg[q] = a.g_hpost ? ld_any(a.g_hpost, tk * N + (f - N), gdt) : 0.f;
        pa[q] = ld_any(a.alpha[1], 0, pdt);
        pb[q] = ld_any(a.bias[1], f - N, pdt);
      } else {
        pg[q] = a.g_hres ? ld_any(a.g_hres, tk * N * N + (f - 2 * N), gdt) : 0.f;
        pa[q] = ld_any(a.alpha[2], 0, pdt);
      }
    }
  }

  const auto rphi = make_rsrc(a.phi, (uint32_t)NC * FD * ES);
  // phi A operand of chunk j, k-tile h, K-step ks: A-row r is column
  // c0 + 8 (r / 4) + 4 h + r % 4 of the chunk, lane group g features 32 ks + 8g .. + 7
  // (fp32 phi: those 8 values, to be split into hi and lo operands).
  auto phi_op = [&](int j, int h, int ks) {
    int ci, c0;
    chunk(j, ci, c0);
    const int col = c0 + 8 * (r >> 2) + 4 * h + (r & 3);
    if constexpr (FD % 8 == 0) {
      const bool ok = col < C && 32 * ks + 8 * g < FD;
      return XV::load(rphi, ok ? (uint32_t)((ci * C + col) * FD + 32 * ks + 8 * g) * ES : kBufOob);
    } else {  // FD in {2, 4} (MHCHead at n = 2, 4; no H_res at n = 2): the row's
              // FD features go to lane group 0, zeros elsewhere
      const bool ok = col < C && g == 0;
      return XV::template load_first<FD>(rphi, ok ? (uint32_t)((ci * C + col) * FD) * ES : kBufOob);
    }
  };

  // ---- gh partials per chunk: sum_c g_sub[c] * x[i][c].  The g_sub loads go
  // out in batches of GB independent loads (one register set each) before
  // they are consumed; one reused register set would wait a round trip each.
  constexpr int GB = KJ < 6 ? KJ : 6;
#pragma unroll
  for (int j0 = 0; j0 < KJ; j0 += GB) {
    XV gvb[GB];
    XV xvb[XRES ? 1 : GB];
    if constexpr (RS) {  // a pair's g_sub: 64 columns of one stream's row (C % 64 == 0)
#pragma unroll
      for (int u = 0; u < GB; u += 2) {
        int ci, c0;
        chunk(j0 + u, ci, c0);
#pragma unroll
        for (int i = 0; i < NRI; ++i) {
          const int tt = RPI * i + lane / PPR;
          const int pc = lane % PPR;
          piece(gvb[u + i / XP], i % XP) =
              buf_load16(rgs, j0 + u < KJ && c0 + pc * (16 / (int)ES) < C ? (uint32_t)(tt * C + c0) * ES + 16u * pc
                                                                          : kBufOob);
        }
      }
#pragma unroll
      for (int u = 0; u < GB; u += 2) {
#pragma unroll
        for (int i = 0; i < NRI; ++i) {
          const int tt = RPI * i + lane / PPR;
          s_rs[wave][tt][(lane % PPR) ^ (tt & 7)] = piece(gvb[u + i / XP], i % XP);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < XP; ++e) piece(gvb[u + h], e) = s_rs[wave][r][(PPR / 2 * h + XP * g + e) ^ (r & 7)];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      }
    } else {
#pragma unroll
      for (int u = 0; u < GB; ++u) {
        int ci, c0;
        chunk(j0 + u, ci, c0);
        const bool ok = j0 + u < KJ && c0 + 8 * g < C;
        gvb[u] = XV::load(rgs, ok ? (uint32_t)(r * C + c0 + 8 * g) * ES : kBufOob);
        if constexpr (!XRES) xvb[u] = j0 + u < KJ ? x_chunk(j0 + u) : XV::load(rx, kBufOob);
      }
    }
#pragma unroll
    for (int u = 0; u < GB; ++u) {
      const int j = j0 + u;
      if (j >= KJ) break;
      const float acc = XV::dot(gvb[u], XRES ? xs[j] : xvb[u]);
      const float a16 = acc + xor_lane16(acc);
      const float a32 = a16 + xor_lane32(a16);
      if (g == 0) s_gp[kidx(j)][r] = a32;
    }
  }
  __syncthreads();

  // ---- gates: g_raw and alpha * g_raw per (token, feature)
#pragma unroll
  for (int q = 0; q < IPT; ++q) {
    const int idx = tid + q * NW * 64;
    if (idx >= GI) break;
    const int tt = idx / (KS * 32);
    const int f = idx - tt * (KS * 32);
    float gm = 0.f;
    if (f < FD && tt < valid) {
      const int64_t tk = t0 + tt;
      const float m = pm[q];
      const float alpha = pa[q];
      float graw;
      if (f < N) {
        float gh = pg[q];
        for (int cb = 0; cb < NCB; ++cb) gh += s_gp[f * NCB + cb][tt];
        const float sg = sigmoid_f(fmaf(alpha, m, pb[q]));
        graw = gh * sg * (1.0f - sg);
        s_hp[tt][f] = sg + a.pre_eps;
      } else if (f < 2 * N) {
        const float sg = sigmoid_f(fmaf(alpha, m, pb[q]));
        graw = pg[q] * sg * (1.0f - sg) * a.post_mult;
      } else {
        graw = pg[q];
      }
      a.g_raw[tk * FD + f] = graw;
      gm = graw * alpha;
    } else if (f < N) {
      s_hp[tt][f] = 0.f;
    }
    s_gm[tt][f] = gm;
    s_mx[tt][f] = f < FD && tt < valid ? pm[q] : 0.f;
  }
  __syncthreads();

  // ---- B operands: lane (token r, g) holds features 32s + 8g .. + 7, hi and lo.
  // The same pass forms mean_k(xn * gxn) without touching x:
  //   sum_k xn[k] gxn[k] = sum_f gm[f] sum_k xn[k] phi[k, f] = sum_f gm[f] mixes_raw[f],
  // the forward's fp32 projection, saved for backward.
  bf16x8_t bhi[KS];
  bf16x8_t blo[KS];
  float msum = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    U32x4 h4, l4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v0 = s_gm[r][32 * ks + 8 * g + 2 * e];
      const float v1 = s_gm[r][32 * ks + 8 * g + 2 * e + 1];
      msum = fmaf(v0, s_mx[r][32 * ks + 8 * g + 2 * e], msum);
      msum = fmaf(v1, s_mx[r][32 * ks + 8 * g + 2 * e + 1], msum);
      const uint32_t hp = pack_bf16x2(v0, v1);
      h4.v[e] = hp;
      l4.v[e] = pack_bf16x2(v0 - bf16lo(hp), v1 - bf16hi(hp));
    }
    bhi[ks] = __builtin_bit_cast(bf16x8_t, h4);
    blo[ks] = __builtin_bit_cast(bf16x8_t, l4);
  }

  msum += xor_lane16(msum);
  msum += xor_lane32(msum);
  const float mean = msum / (float)NC;  // mean_k(xn * gxn)

  // ---- gxn = phi . (alpha * g_raw) on MFMA, and
  //      g_x = inv * (gxn - xn * mean) + h_pre[i] * g_sub.
  // Where phi is one K-step wide (FD <= 32), a chunk's phi A operands and its
  // g_sub go out three chunks ahead (four register sets: 123 VGPRs at n = 4,
  // C = 768, within two 8-wave workgroups per CU; one ahead at 16 chunks a
  // wave), so the MFMAs and the g_x
  // arithmetic of chunk j run while the loads of chunks j + 1 .. j + 3 are in
  // flight instead of each load being waited for in turn (C2 68.0 -> 67.3 us
  // against one chunk ahead).  Wider phi (n = 8, full)
  // keeps one set, loaded at the start of its chunk (CH: one round trip a
  // chunk) up to 12 chunks a wave, and operand by operand beyond that (the
  // whole set would spill).
  constexpr bool PF = KS == 1;
  constexpr bool CH = !PF && KJ <= 12;
  struct ChunkIn {
    XV av[PB ? 1 : 2][PB ? 1 : KS];
    U32x4 pb[PB ? 2 : 1][PB ? NPBH : 1];  // PB: the chunk's phi block, 16-byte pieces along the lanes
    XV gv;
    XV xv[XRES ? 1 : 1];  // the chunk's x when it is not held from the start
  };
  auto load_chunk = [&](int j, ChunkIn& in) {
    int ci, c0;
    chunk(j, ci, c0);
    if constexpr (PB) {
      const uint32_t base = (uint32_t)((ci * C + c0) * FD) * ES;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < NPBH; ++i) {
          const int ph = 64 * i + lane;
          const int q = ph / GPC;
          const uint32_t off = base + (uint32_t)((8 * q + 4 * h) * FD) * ES + 16u * (ph - q * GPC);
          // C % 8 == 0: a 4-row group lies wholly inside or wholly past C
          in.pb[h][i] = buf_load16(rphi, c0 + 8 * q < C && ph < NPH ? off : kBufOob);
        }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) in.av[h][ks] = phi_op(j, h, ks);
    }
    const bool ok = c0 + 8 * g < C;
    in.gv = XV::load(rgs, ok ? (uint32_t)(r * C + c0 + 8 * g) * ES : kBufOob);
    if constexpr (!XRES) in.xv[0] = x_chunk(j);
  };
  // 16 chunks a wave, or x streamed with the chunk: four sets would spill
  constexpr int PD = PF ? (KJ <= 12 && XRES ? 4 : 2) : 1;
  ChunkIn cin[PD];
  if constexpr (PF) {
#pragma unroll
    for (int p = 0; p < PD - 1; ++p)
      if (p < KJ) load_chunk(p, cin[p]);
  }
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    ChunkIn& cur = cin[PF ? (j % PD) : 0];
    if constexpr (PF) {
      if (j + PD - 1 < KJ) load_chunk(j + PD - 1, cin[(j + PD - 1) % PD]);
    } else if constexpr (CH) {
      load_chunk(j, cur);
    }
    int ci, c0;
    chunk(j, ci, c0);
    const bool ok = c0 + 8 * g < C;
    // PB: A-row r of half h is row r % 4 of group r / 4 of that half; lane
    // group g takes features 32 ks + 8g .. + 7, pieces (4 ks + g) XP .. + XP - 1
    // of the row
    XV avb[PB ? 2 : 1][PB ? KS : 1];
    auto pb_stage = [&](int h) {
#pragma unroll
      for (int i = 0; i < NPBH; ++i)
        if (64 * i + lane < NPH) s_pb[wave][(PBH ? 0 : h) * NPH + 64 * i + lane] = cur.pb[h][i];
    };
    auto pb_fetch = [&](int h) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int p0 = (PBH ? 0 : h) * NPH + (r >> 2) * GPC + (r & 3) * (FD * XP / 8) + 4 * XP * ks + XP * g;
#pragma unroll
        for (int e = 0; e < XP; ++e)
          piece(avb[h][ks], e) = 32 * ks + 8 * g < FD ? s_pb[wave][p0 + e] : U32x4{{0u, 0u, 0u, 0u}};
      }
    };
    if constexpr (PB && !PBH) {
      pb_stage(0);
      pb_stage(1);
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      pb_fetch(0);
      pb_fetch(1);
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    f32x4_t d2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (PB && PBH) {
        pb_stage(h);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        pb_fetch(h);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      }
      f32x4_t d = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const XV av = PB ? avb[PB ? h : 0][PB ? ks : 0] : (PF || CH ? cur.av[PB ? 0 : h][PB ? 0 : ks] : phi_op(j, h, ks));
        if constexpr (F32) {  // phi_hi . (b_hi + b_lo) + phi_lo . b_hi
          const bf16x8_t ahi = XV::hi(av);
          const bf16x8_t alo = XV::lo(av);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bhi[ks], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, blo[ks], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bhi[ks], d, 0, 0, 0);
        } else {
          const bf16x8_t ab = XV::hi(av);  // bf16 phi: the operand itself
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, bhi[ks], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, blo[ks], d, 0, 0, 0);
        }
      }
      d2[h] = d;
    }
    const XV gv = PF || CH ? cur.gv : XV::load(rgs, ok ? (uint32_t)(r * C + c0 + 8 * g) * ES : kBufOob);
    XV xj;
    if constexpr (XRES) xj = xs[j];
    else xj = PF || CH ? cur.xv[0] : x_chunk(j);
    const float hp = s_hp[r][ci];
    float v[8];
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {  // column 8g + cc
      const float gx = d2[cc >> 2][cc & 3];
      v[cc] = inv * (gx - XV::get(xj, cc) * inv * mean) + hp * XV::get(gv, cc);
    }
    // whole offset in the vector offset, scalar offset the literal 0 (a
    // 128-bit store reads its data registers after issue)
    if constexpr (RS) {  // both chunks of the pair through LDS, then NRI row stores
      U32x4 o[XP];
#pragma unroll
      for (int e = 0; e < 4 * XP; ++e) {
        if constexpr (F32) o[e >> 2].v[e & 3] = __float_as_uint(v[e]);
        else o[0].v[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
      }
#pragma unroll
      for (int e = 0; e < XP; ++e) s_rs[wave][r][(PPR / 2 * (j & 1) + XP * g + e) ^ (r & 7)] = o[e];
      if (j & 1) {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const int col = 64 * (wave + NW * (j >> 1));
#pragma unroll
        for (int i = 0; i < NRI; ++i) {
          const int tt = RPI * i + lane / PPR;
          const int pc = lane % PPR;
          buf_store16(rgx, col + pc * (16 / (int)ES) < NC ? (uint32_t)(tt * NC + col) * ES + 16u * pc : kBufOob,
                      s_rs[wave][tt][pc ^ (tt & 7)]);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      }
    } else {
      XV::store(rgx, ok ? (uint32_t)(r * NC + ci * C + c0 + 8 * g) * ES : kBufOob, v);
    }
  }
}

// Chunks per wave instantiated: 2 .. 16 in steps that cover C <= 1024 for
// n in {2, 4} (8 waves) and n = 8 (16 waves, bf16 only).
template <int N, int MODE, int NW, int KJ, bool F32>
static hipError_t launch_pre_bwd_inst(const PreBwdArgs& a, hipStream_t s) {
  if constexpr (kPreBwdRowPieces && (!F32 || N <= 4) && KJ % 2 == 0) {
    if (a.C % 64 == 0) {  // a chunk pair's 64 columns in one stream's row
      hipLaunchKernelGGL((pre_bwd_mfma_kernel<N, MODE, NW, KJ, F32, true>), dim3((unsigned)((a.M + 15) / 16)),
                         dim3(NW * 64), 0, s, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((pre_bwd_mfma_kernel<N, MODE, NW, KJ, F32>), dim3((unsigned)((a.M + 15) / 16)),
                     dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

template <int N, int MODE, int NW, bool F32, int... KJS>
static hipError_t launch_pre_bwd_mfma_kj(const PreBwdArgs& a, int kj, hipStream_t s) {
  hipError_t r = hipErrorInvalidValue;
  bool done = false;
  ((!done && KJS >= kj ? (r = launch_pre_bwd_inst<N, MODE, NW, KJS, F32>(a, s), done = true) : false), ...);
  return r;
}

template <int N, int MODE, bool F32>
static hipError_t launch_pre_bwd_mfma_mode(const PreBwdArgs& a, hipStream_t s) {
  constexpr int NW = N >= 8 ? 16 : 8;
  const int nch = N * ((a.C + 31) / 32);
  const int kj = (nch + NW - 1) / NW;
  return launch_pre_bwd_mfma_kj<N, MODE, NW, F32, 2, 4, 6, 8, 12, 16>(a, kj, s);
}

// Shapes with an MFMA kernel: x / phi / gradients all bf16 (n in {2, 4, 8}) or
// all fp32 (n in {2, 4}: the fp32 chunks take twice the registers), FD a
// multiple of 8 (whole 8-feature phi operands), C % 8 == 0 and C <= 1024,
// 16-byte aligned x / g_sub / g_x / phi.
static bool pre_bwd_mfma_ok(const PreBwdArgs& a) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (a.mode == kRms) return false;
  const bool bf = a.x_dtype == kBF16 && a.phi_dtype == kBF16 && a.grad_dtype == kBF16;
  const bool f32 = a.x_dtype == kF32 && a.phi_dtype == kF32 && a.grad_dtype == kF32;
  if (!((bf || f32) && (a.n == 2 || a.n == 4 || a.n == 8))) return false;
  const int fd = mode_fd(a.mode, a.n);
  if (fd % 8 != 0 && fd != 4 && fd != 2) return false;  // whole 8-feature operands, or one short one
  if (a.C % 8 != 0 || a.C > 32 * kMfmaMaxColBlocks) return false;
  if ((int64_t)a.n * a.C * mode_fd(a.mode, a.n) * dtype_bytes(a.x_dtype) > 0x7fffffffLL) return false;
  return al(a.x) && al(a.phi) && al(a.g_x) && (a.g_sub == nullptr || al(a.g_sub));
}

template <int N, bool F32>
static hipError_t launch_pre_bwd_mfma_n(const PreBwdArgs& a, hipStream_t s) {
  switch (a.mode) {
    case kFull: return launch_pre_bwd_mfma_mode<N, kFull, F32>(a, s);
    case kNoHres: return launch_pre_bwd_mfma_mode<N, kNoHres, F32>(a, s);
    case kHead: return launch_pre_bwd_mfma_mode<N, kHead, F32>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pre_bwd(const PreBwdArgs& a, hipStream_t s) {
  if (pre_bwd_mfma_ok(a)) {
    if (a.x_dtype == kF32) {
      switch (a.n) {
        case 2: return launch_pre_bwd_mfma_n<2, true>(a, s);
        case 4: return launch_pre_bwd_mfma_n<4, true>(a, s);
        case 8: return launch_pre_bwd_mfma_n<8, true>(a, s);
        default: break;
      }
    } else {
      switch (a.n) {
        case 2: return launch_pre_bwd_mfma_n<2, false>(a, s);
        case 4: return launch_pre_bwd_mfma_n<4, false>(a, s);
        case 8: return launch_pre_bwd_mfma_n<8, false>(a, s);
        default: break;
      }
    }
  }
  hipLaunchKernelGGL(pre_bwd_generic_kernel, dim3((unsigned)a.M), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ----------------------------------------------------------- weight gradients
// Token ranges: R partial sums of every (k, f) in the workspace, then one
// reduction.  Workspace layout (fp32): W[R][n*C][FD], then AB[R][2][FD]
// (sum g_raw, sum g_raw * mixes).
static int weight_ranges(int64_t M) {
  const int64_t r = (M + 255) / 256;
  return (int)(r < 1 ? 1 : (r > 64 ? 64 : r));
}

int64_t weights_range_bytes(int n, int C, int mode) {
  const int FD = mode_fd(mode, n);
  return ((int64_t)n * C * FD + 2 * (int64_t)FD) * 4;
}

int64_t weights_workspace_bytes(int64_t M, int n, int C, int mode) {
  return weight_ranges(M) * weights_range_bytes(n, C, mode);
}

__global__ __launch_bounds__(256) void weights_partial_generic_kernel(WeightsArgs a, int R, int64_t per) {
  const int FD = mode_fd(a.mode, a.n);
  const int64_t NC = (int64_t)a.n * a.C;
  const int r = blockIdx.x;
  const int64_t q = (int64_t)blockIdx.y * 256 + threadIdx.x;
  const int64_t t0 = (int64_t)r * per;
  const int64_t t1 = t0 + per < a.M ? t0 + per : a.M;
  if (q < NC * FD) {
    const int64_t k = q / FD;
    const int f = (int)(q - k * FD);
    float acc = 0.f;
    for (int64_t t = t0; t < t1; ++t)
      acc = fmaf(ld_any(a.x, t * NC + k, a.x_dtype) * a.inv_rms[t], a.g_raw[t * FD + f], acc);
    a.work[(r * NC + k) * FD + f] = acc;
  }
  if (blockIdx.y == 0) {  // alpha / bias partials of this range (FD = 288 at n = 16)
    for (int f = threadIdx.x; f < FD; f += 256) {
      float sb = 0.f, sa = 0.f;
      for (int64_t t = t0; t < t1; ++t) {
        const float gr = a.g_raw[t * FD + f];
        sb += gr;
        sa = fmaf(gr, a.mixes[t * FD + f], sa);
      }
      float* ab = a.work + (int64_t)R * NC * FD + (int64_t)r * 2 * FD;
      ab[f] = sb;
      ab[FD + f] = sa;
    }
  }
}

__device__ __forceinline__ int seg_of(int f, int n) { return f < n ? 0 : (f < 2 * n ? 1 : 2); }

// Sum of w[r * stride], r < R (R <= 64, at most 64 token ranges), in a fixed
// order: batches of 16 independent loads (so a thread waits for one memory
// round trip per batch, not one per range), each summed as a pairwise tree.
// Slots past R load nothing (R is uniform: a scalar branch, no divergence).
constexpr int kRangeBatch = 16;
__device__ __forceinline__ float sum_ranges(const float* __restrict__ w, int64_t stride, int R) {
  float total = 0.f;
  for (int r0 = 0; r0 < R; r0 += kRangeBatch) {
    float v[kRangeBatch];
#pragma unroll
    for (int u = 0; u < kRangeBatch; ++u) v[u] = r0 + u < R ? w[(int64_t)(r0 + u) * stride] : 0.f;
#pragma unroll
    for (int h = kRangeBatch / 2; h > 0; h >>= 1)
#pragma unroll
      for (int u = 0; u < h; ++u) v[u] += v[u + h];
    total += v[0];
  }
  return total;
}

// The same over four consecutive elements: 16-byte loads of each range's
// partials, the same order of sums per element.
__device__ __forceinline__ f32x4_t sum_ranges4(const float* __restrict__ w, int64_t stride, int R) {
  f32x4_t total = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int r0 = 0; r0 < R; r0 += kRangeBatch) {
    f32x4_t v[kRangeBatch];
#pragma unroll
    for (int u = 0; u < kRangeBatch; ++u)
      v[u] = r0 + u < R ? *reinterpret_cast<const f32x4_t*>(w + (int64_t)(r0 + u) * stride)
                        : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = kRangeBatch / 2; h > 0; h >>= 1)
#pragma unroll
      for (int u = 0; u < h; ++u) v[u] += v[u + h];
    total += v[0];
  }
  return total;
}

// Grid: one thread per phi element (V4: per four consecutive elements), plus
// one last workgroup for the alpha / bias sums (one thread per (feature,
// kind)).
template <bool V4>
__global__ __launch_bounds__(256) void weights_reduce_kernel(WeightsArgs a, int R) {
  const int n = a.n;
  const int FD = mode_fd(a.mode, n);
  const int64_t NC = (int64_t)n * a.C;
  const int64_t q = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * (V4 ? 4 : 1);
  if (blockIdx.x + 1 < gridDim.x) {
    // The three segments' alphas, loaded before the partials with no branch
    // and converted after the sums: read per element after the sums (a
    // per-lane alpha pointer, then a per-dtype branch), they were a chain of
    // round trips at the end of every thread.
    uint32_t alw[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) alw[k] = ld_bits(a.alpha[k], 1, 0, a.param_dtype, a.alpha[k] != nullptr);
    auto alpha_of = [&](int f) {
      const int sg = seg_of(f, n);
      return bits_to_f32(sg == 0 ? alw[0] : (sg == 1 ? alw[1] : alw[2]), a.param_dtype);
    };
    if (q < NC * FD) {
      if constexpr (V4) {
        const f32x4_t acc = sum_ranges4(a.work + q, NC * FD, R);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[e] * alpha_of((int)((q + e) % FD));
        if (a.phi_dtype == kF32) {
          *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.g_phi) + q) = f32x4_t{v[0], v[1], v[2], v[3]};
        } else {
          uint32_t w2[2];
#pragma unroll
          for (int h = 0; h < 2; ++h)
            w2[h] = a.phi_dtype == kBF16
                        ? (uint32_t)f32_to_bf16_bits(v[2 * h]) | ((uint32_t)f32_to_bf16_bits(v[2 * h + 1]) << 16)
                        : (uint32_t)f32_to_f16_bits(v[2 * h]) | ((uint32_t)f32_to_f16_bits(v[2 * h + 1]) << 16);
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.g_phi) + q) = make_uint2(w2[0], w2[1]);
        }
      } else {
        const int f = (int)(q % FD);
        const float acc = sum_ranges(a.work + q, NC * FD, R);
        st_any(a.g_phi, q, a.phi_dtype, acc * alpha_of(f));
      }
    }
  } else {
    __shared__ float s_a[kMaxFD];
    const float* ab = a.work + (int64_t)R * NC * FD;
    for (int t = threadIdx.x; t < 2 * FD; t += blockDim.x) {  // t < FD: bias (sum g_raw), else alpha
      const int f = t < FD ? t : t - FD;               // (sum g_raw * mixes)
      const float v = sum_ranges(ab + t, 2 * FD, R);
      if (t < FD) {
        const int sg = seg_of(f, n);
        const int base = sg == 0 ? 0 : (sg == 1 ? n : 2 * n);
        if (a.g_bias[sg]) st_any(a.g_bias[sg], f - base, a.param_dtype, v);
      } else {
        s_a[f] = v;
      }
    }
    __syncthreads();
    if (threadIdx.x < 3) {
      const int sg = threadIdx.x;
      const int lo = sg == 0 ? 0 : (sg == 1 ? n : 2 * n);
      const int hi = sg == 0 ? n : (sg == 1 ? 2 * n : 2 * n + n * n);
      if (hi <= FD && a.g_alpha[sg]) {
        float sa = 0.f;
        for (int f = lo; f < hi; ++f) sa += s_a[f];
        st_any(a.g_alpha[sg], 0, a.param_dtype, sa);
      }
    }
  }
}

// bf16 or fp32 x on MFMA.  Workgroup (k-slice of 128 MT columns, token
// range): per step of 64 tokens the x tile is written to LDS transposed
// ([column][token], two tokens per 32-bit write) and u = inv_rms * g_raw
// ([feature][token]) split into bf16 hi + lo, then wave w accumulates, for
// its MT 16-column tiles m (columns 16 (w + 8m) + i),
//   D[16(w + 8m) + i][f] += sum_t x[t][k0 + 16(w + 8m) + i] * u[t][f]
// with A = x^T rows (16-byte LDS reads of 8 tokens) and B = u columns, each
// B operand read once for the MT tiles (the per-step u work and its LDS
// reads are per workgroup, so wider slices spend less of them per column).  An
// fp32 x is split the same way (a second transposed tile holds x_lo) and
// three products run per step: x_hi u_hi + x_hi u_lo + x_lo u_hi.
// One more workgroup per token range (blockIdx.x == the slice count) sums
// g_raw and g_raw * mixes per feature over the range: the alpha / bias
// partials, kept off the slices' registers.
constexpr int kWTok = 64;                // tokens per step
constexpr int kWCols = 128;              // columns per workgroup and 16-column tile per wave
constexpr int kWRow = kWTok * 2 + 16;    // LDS row stride in bytes (64 bf16 + pad)

// The alpha / bias partials of one token range [tb, te): thread (row, quad)
// sums features 4 quad .. 4 quad + 3 over tokens tb + row, tb + row + rows,
// ..., four tokens in flight; the rows are then summed in order.
__device__ __forceinline__ void weights_ab_range(const WeightsArgs& a, int FD, int64_t tb, int64_t te,
                                                 float* ab, float (*s_red)[2][4]) {
  const int tid = threadIdx.x;
  const int Q = (FD + 3) / 4;
  const int rows = 512 / Q;
  const int row = tid / Q;
  const int q = tid % Q;
  const uint32_t span = (uint32_t)((te - tb) * FD * 4);
  const auto rg = make_rsrc(a.g_raw + tb * FD, span);
  const auto rm = make_rsrc(a.mixes + tb * FD, span);
  float sb[4] = {0.f, 0.f, 0.f, 0.f}, sa[4] = {0.f, 0.f, 0.f, 0.f};
  auto quad = [&](__amdgpu_buffer_rsrc_t r, int64_t t) -> U32x4 {  // FD % 4 == 0
    return buf_load16(r, t < te - tb ? (uint32_t)(t * FD * 4) + 16u * q : kBufOob);
  };
  if (row < rows) {
    for (int64_t t = row; t < te - tb; t += 4 * (int64_t)rows) {  // uniform per thread
      U32x4 g[4], m[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        g[j] = quad(rg, t + (int64_t)j * rows);
        m[j] = quad(rm, t + (int64_t)j * rows);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gv = __uint_as_float(g[j].v[e]);
          sb[e] += gv;
          sa[e] = fmaf(gv, __uint_as_float(m[j].v[e]), sa[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s_red[tid][0][e] = sb[e];
      s_red[tid][1][e] = sa[e];
    }
  }
  __syncthreads();
  for (int f = tid; f < FD; f += 512) {
    float b = 0.f, al = 0.f;
    for (int r = 0; r < rows; ++r) {
      b += s_red[r * Q + f / 4][0][f % 4];
      al += s_red[r * Q + f / 4][1][f % 4];
    }
    ab[f] = b;
    ab[FD + f] = al;
  }
}

// x is loaded PF steps ahead and the per-token values TD steps ahead (step
// t + TD's go out as soon as step t has consumed its own).  Per-token items
// are (token pair, feature quad): 16-byte loads of both tokens' g_raw quads
// and one inv_rms each, token pairs along the lanes so the u writes to LDS
// fill whole rows.
template <int NTF, bool F32, int MT, int PF, int TD, int WPE>  // feature tiles, fp32 x, column tiles a wave,
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPE)))  // x / per-token steps in flight,
void weights_mfma_kernel(WeightsArgs a, int64_t per) {                       // waves / SIMD
  constexpr int F16 = NTF * 16;
  constexpr int QT = F16 / 4;                   // feature quads of the tile
  constexpr int NI = (32 * QT + 511) / 512;     // (token pair, quad) items per thread
  constexpr int XQ = F32 ? 2 : 1;  // 16-byte loads per 8 columns of one token
  constexpr uint32_t ES = F32 ? 4u : 2u;
  constexpr int WC = kWCols * MT;  // columns of the slice
  __shared__ __attribute__((aligned(16))) unsigned char s_x[WC * kWRow];
  __shared__ __attribute__((aligned(16))) unsigned char s_xl[F32 ? WC * kWRow : 16];
  __shared__ __attribute__((aligned(16))) unsigned char s_uh[F16 * kWRow];
  __shared__ __attribute__((aligned(16))) unsigned char s_ul[F16 * kWRow];
  const int FD = mode_fd(a.mode, a.n);
  const int NC = a.n * a.C;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int rng = blockIdx.y;
  const int64_t tb = (int64_t)rng * per;
  const int64_t te = tb + per < a.M ? tb + per : a.M;
  if (blockIdx.x + 1 == gridDim.x) {  // the range's alpha / bias partials
    static_assert(512 * 2 * 4 * 4 <= kWCols * kWRow, "reduction rows fit s_x");
    weights_ab_range(a, FD, tb, te, a.work + (int64_t)gridDim.y * NC * FD + (int64_t)rng * 2 * FD,
                     reinterpret_cast<float (*)[2][4]>(s_x));
    return;
  }
  const int k0 = blockIdx.x * WC;

  // x: 8-column groups kc + 16m (columns k0 + 8 (kc + 16m) .. + 7) of token
  // pair tp (tokens 2tp, 2tp + 1 of the step).  Sixteen consecutive lanes
  // cover 256 bytes of a token's row, so each wave load reads whole 128-byte
  // lines.
  const int kc = tid & 15;
  const int tp = tid >> 4;
  // In s_x the 16-byte groups of token pairs (4 pairs = 8 tokens) of column
  // group kc are XOR-permuted by kc & 7: the transposed writes of 16 column
  // groups at one token pair then spread over 8 bank groups instead of one,
  // and an MFMA read of 8 consecutive tokens stays one aligned 16-byte read.
  auto tp_slot = [](int pair, int group) { return pair ^ (4 * (group & 7)); };

  // Per-token items: item i of this thread is token pair pp = idx % 32 and
  // feature quad fq = idx / 32 (idx = tid + 512 i; fq < QT), read through
  // descriptors over the range (tokens past te read zeros).
  const auto rg = make_rsrc(a.g_raw + tb * FD, (uint32_t)((te - tb) * FD * 4));
  const auto ri = make_rsrc(a.inv_rms + tb, (uint32_t)((te - tb) * 4));
  struct XStep {  // a step's x, PF steps ahead
    U32x4 xa[MT][XQ], xb[MT][XQ];
  };
  struct Step {  // a step's per-token values, one step ahead
    U32x4 ga[NI], gb[NI];
    float ia[NI], ib[NI];
  };
  auto load_x = [&](int64_t t, XStep& st) {
    const int valid = t < te ? (int)(te - t < kWTok ? te - t : kWTok) : 0;
    const auto rs = make_rsrc(static_cast<const unsigned char*>(a.x) + (t < te ? t : 0) * NC * ES,
                              (uint32_t)valid * NC * ES);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int col = k0 + 8 * (kc + 16 * m);
      const bool okc = col < NC;
#pragma unroll
      for (int h = 0; h < XQ; ++h) {
        st.xa[m][h] = buf_load16_nt(rs, okc ? (uint32_t)((2 * tp) * NC + col) * ES + 16u * h : kBufOob, 0);
        st.xb[m][h] = buf_load16_nt(rs, okc ? (uint32_t)((2 * tp + 1) * NC + col) * ES + 16u * h : kBufOob, 0);
      }
    }
  };
  // Quad fq of token tok (relative to tb; FD % 4 == 0, the launcher keeps
  // (per + 64) * FD * 4 below 2^31, and tokens past te land past the descriptor).
  auto g_quad = [&](bool live, uint32_t tok, int fq) -> U32x4 {
    return buf_load16(rg, oob_unless(live && 4 * fq < FD, tok * (uint32_t)FD * 4u + 16u * fq));
  };
  auto load_step = [&](int64_t t, Step& st) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int idx = tid + 512 * i;
      const int pp = idx & 31;
      const int fq = idx >> 5;
      const uint32_t ta = (uint32_t)(t - tb) + 2u * pp;
      const bool live = fq < QT && t < te;
      st.ga[i] = g_quad(live, ta, fq);
      st.gb[i] = g_quad(live, ta + 1, fq);
      st.ia[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ri, (int)oob_unless(live, 4u * ta), 0, 0));
      st.ib[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ri, (int)oob_unless(live, 4u * ta + 4u), 0, 0));
    }
  };
  f32x4_t acc[MT][NTF];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int ft = 0; ft < NTF; ++ft) acc[m][ft] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One step: the staged loads to LDS, then the MFMAs while later steps load.
  auto run_step = [&](int64_t t, XStep& xc, Step& cur) {
    // u = inv * g_raw as hi / lo bf16 token pairs, [feature][token]
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int idx = tid + 512 * i;
      const int pp = idx & 31;
      const int fq = idx >> 5;
      if (fq < QT) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float va = cur.ia[i] * __uint_as_float(cur.ga[i].v[e]);
          const float vb = cur.ib[i] * __uint_as_float(cur.gb[i].v[e]);
          const uint32_t hi = pack_bf16x2(va, vb);
          const int off = (4 * fq + e) * kWRow + pp * 4;
          *reinterpret_cast<uint32_t*>(s_uh + off) = hi;
          *reinterpret_cast<uint32_t*>(s_ul + off) = pack_bf16x2(va - bf16lo(hi), vb - bf16hi(hi));
        }
      }
    }
    // Step t + TD's per-token values go out as soon as these are consumed.
    load_step(t + TD * kWTok, cur);
    // x tile transposed: column 8 (kc + 16m) + e, tokens (2tp, 2tp + 1) in one dword
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t off = (8 * (kc + 16 * m) + e) * kWRow + tp_slot(tp, kc) * 4;
        if constexpr (F32) {
          const float va = __uint_as_float(xc.xa[m][e >> 2].v[e & 3]);
          const float vb = __uint_as_float(xc.xb[m][e >> 2].v[e & 3]);
          const uint32_t hi = pack_bf16x2(va, vb);
          *reinterpret_cast<uint32_t*>(s_x + off) = hi;
          *reinterpret_cast<uint32_t*>(s_xl + off) = pack_bf16x2(va - bf16lo(hi), vb - bf16hi(hi));
        } else {
          const uint32_t wa = xc.xa[m][0].v[e >> 1];
          const uint32_t wb = xc.xb[m][0].v[e >> 1];
          const uint32_t d = (e & 1) ? ((wa >> 16) | (wb & 0xffff0000u)) : ((wa & 0xffffu) | (wb << 16));
          *reinterpret_cast<uint32_t*>(s_x + off) = d;
        }
      }
    __syncthreads();
    // x of step t + PF flies over the MFMAs (issued after the per-token values
    // of step t + 1: the vector-memory counter retires in order).
    load_x(t + PF * kWTok, xc);
#pragma unroll
    for (int ks = 0; ks < kWTok / 32; ++ks) {
      bf16x8_t av[MT];
      int xoff[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const int xc = 16 * (wave + 8 * m) + r;  // column of the slice
        xoff[m] = xc * kWRow + tp_slot(16 * ks + 4 * g, xc >> 3) * 4;
        av[m] = *reinterpret_cast<const bf16x8_t*>(s_x + xoff[m]);
      }
#pragma unroll
      for (int ft = 0; ft < NTF; ++ft) {
        const int off = (16 * ft + r) * kWRow + (32 * ks + 8 * g) * 2;
        const bf16x8_t uh = *reinterpret_cast<const bf16x8_t*>(s_uh + off);
        const bf16x8_t ul = *reinterpret_cast<const bf16x8_t*>(s_ul + off);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          acc[m][ft] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[m], uh, acc[m][ft], 0, 0, 0);
          acc[m][ft] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[m], ul, acc[m][ft], 0, 0, 0);
          if constexpr (F32)
            acc[m][ft] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                *reinterpret_cast<const bf16x8_t*>(s_xl + xoff[m]), uh, acc[m][ft], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  };
  constexpr int U = PF * TD / (PF % TD == 0 || TD % PF == 0 ? (PF < TD ? PF : TD) : 1);  // lcm
  XStep st[PF];
  Step tk[TD];
#pragma unroll
  for (int q = 0; q < TD; ++q) load_step(tb + q * kWTok, tk[q]);
#pragma unroll
  for (int q = 0; q < PF; ++q) load_x(tb + q * kWTok, st[q]);
  for (int64_t t = tb; t < te; t += U * kWTok) {  // uniform; steps past te read nothing
#pragma unroll
    for (int q = 0; q < U; ++q)
      if (t + q * kWTok < te) run_step(t + q * kWTok, st[q % PF], tk[q % TD]);
  }
  // partial W of this range: lane (feature column r, g) holds rows 4g .. 4g + 3
  // of each of its column tiles
  float* W = a.work + (int64_t)rng * NC * FD;
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int ft = 0; ft < NTF; ++ft)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + 16 * (wave + 8 * m) + 4 * g + j;
        const int f = 16 * ft + r;
        if (k < NC && f < FD) W[(int64_t)k * FD + f] = acc[m][ft][j];
      }
}

// Column tiles a wave (MT), steps of x (PF) and of the per-token values (TD)
// in flight, and the waves per SIMD each instance is held to.  Measured at
// 16384 tokens, n = 4 and 8192 tokens, n = 8 (C = 768; partials + reduction):
//   bf16, FD <= 32: MT 1, PF 2, TD 2 at two workgroups a CU (29.2 us; 256-column
//     slices 31.2 us: the step's chain of waits and barriers bounds it, not
//     the per-column work they halve);
//   bf16, FD > 32: MT 2, PF 2, TD 2 at one workgroup a CU (41.0 us; MT 1 at two
//     a CU 50.3 us, with x one step ahead 65.8 us);
//   fp32 x: PF 2, TD 1, and MT 2 with PF 1 where FD > 32 (C2 54.3 us, C5 67.7 us).
template <int NTF, bool F32>
constexpr int weights_mt() {
  return NTF >= 3 ? 2 : 1;
}
template <int NTF, bool F32>
constexpr int weights_pf() {
  return F32 && NTF >= 3 ? 1 : 2;
}
template <int NTF, bool F32>
constexpr int weights_td() {
  return !F32 ? 2 : 1;
}
template <int NTF, bool F32>
constexpr int weights_wpe() {
  return NTF >= 3 ? 2 : 4;
}
#define WEIGHTS_INST(NTF, F32)                                                                           \
  weights_mfma_kernel<NTF, F32, weights_mt<NTF, F32>(), weights_pf<NTF, F32>(), weights_td<NTF, F32>(), \
                      weights_wpe<NTF, F32>()>

// Workgroups of weights_mfma_kernel<NTF, F32> one CU holds at once (from its
// registers and LDS; cached per instance).
template <int NTF, bool F32>
static int weights_wg_per_cu() {
  static int cached = 0;
  if (cached == 0) {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, WEIGHTS_INST(NTF, F32), 512, 0) != hipSuccess ||
        blocks < 1)
      blocks = 1;
    cached = blocks;
  }
  return cached;
}

template <int NTF>
static int weights_wg_per_cu(const WeightsArgs& a) {
  return a.x_dtype == kF32 ? weights_wg_per_cu<NTF, true>() : weights_wg_per_cu<NTF, false>();
}

// Columns of one workgroup's slice for the instance a launch takes.
template <int NTF>
static int weights_slice_cols(const WeightsArgs& a) {
  return kWCols * (a.x_dtype == kF32 ? weights_mt<NTF, true>() : weights_mt<NTF, false>());
}

template <int NTF>
static hipError_t launch_weights_mfma(const WeightsArgs& a, int R, int64_t per, hipStream_t s) {
  const int NC = a.n * a.C;
  const int wc = weights_slice_cols<NTF>(a);
  const dim3 grid((unsigned)((NC + wc - 1) / wc + 1), (unsigned)R);  // + the alpha / bias workgroup
  if (a.x_dtype == kF32)
    hipLaunchKernelGGL((WEIGHTS_INST(NTF, true)), grid, dim3(512), 0, s, a, per);
  else
    hipLaunchKernelGGL((WEIGHTS_INST(NTF, false)), grid, dim3(512), 0, s, a, per);
  return hipGetLastError();
}

hipError_t launch_pre_bwd_weights(const WeightsArgs& a, hipStream_t s) {
  const int FD = mode_fd(a.mode, a.n);
  const int64_t NC = (int64_t)a.n * a.C;
  const int64_t qb = (NC * FD + 255) / 256;
  const int ntf = (FD + 15) / 16;
  // The MFMA kernel reads g_raw and mixes as 16-byte feature quads (FD % 4 == 0:
  // every mode but MHCHead at n = 2) at 32-bit per-range offsets: (per + 64) * FD
  // * 4 < 2^31 with per <= M (up to 6.7 M tokens at FD = 80 in one range).
  const bool mfma = (a.x_dtype == kBF16 || a.x_dtype == kF32) && NC % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                    ((reinterpret_cast<uintptr_t>(a.g_raw) | reinterpret_cast<uintptr_t>(a.mixes)) & 15) == 0 &&
                    FD % 4 == 0 && (a.M + kWTok) * FD * 4 < ((int64_t)1 << 31) &&
                    (ntf == 1 || ntf == 2 || ntf == 3 || ntf == 5);  // FD <= 80 (LDS)
  int R = weight_ranges(a.M);
  if (a.max_ranges > 0 && R > a.max_ranges) R = a.max_ranges;  // smaller workspace
  hipError_t e;
  if (mfma) {
    // Token ranges of whole 64-token steps, as many as one round of
    // workgroups holds (every CU as full as the kernel's registers and LDS
    // allow; two rounds if one round leaves fewer than four ranges), so no
    // short last round of stragglers follows the full ones.
    int wpc = 1, wc = kWCols;
    switch (ntf) {
      case 1: wpc = weights_wg_per_cu<1>(a); wc = weights_slice_cols<1>(a); break;
      case 2: wpc = weights_wg_per_cu<2>(a); wc = weights_slice_cols<2>(a); break;
      case 3: wpc = weights_wg_per_cu<3>(a); wc = weights_slice_cols<3>(a); break;
      default: wpc = weights_wg_per_cu<5>(a); wc = weights_slice_cols<5>(a); break;
    }
    const int64_t slices = (NC + wc - 1) / wc + 1;  // + the alpha / bias workgroup
    const int64_t cap = (int64_t)wpc * device_cus();
    int64_t want = cap / slices;
    if (want < 4) want = 2 * cap / slices;
    if (want < 1) want = 1;
    if (want < R) R = (int)want;
    int64_t per = (a.M + R - 1) / R;
    per = (per + kWTok - 1) / kWTok * kWTok;
    R = (int)((a.M + per - 1) / per);
    switch (ntf) {
      case 1: e = launch_weights_mfma<1>(a, R, per, s); break;
      case 2: e = launch_weights_mfma<2>(a, R, per, s); break;
      case 3: e = launch_weights_mfma<3>(a, R, per, s); break;
      case 5: e = launch_weights_mfma<5>(a, R, per, s); break;
      default: e = launch_weights_mfma<5>(a, R, per, s); break;
    }
  } else {
    const int64_t per = (a.M + R - 1) / R;
    hipLaunchKernelGGL(weights_partial_generic_kernel, dim3((unsigned)R, (unsigned)qb), dim3(256), 0, s,
                       a, R, per);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  // Four phi elements a thread where whole 16-byte groups of partials line up
  // (the workspace is the caller's allocation: checked, not assumed) and there
  // are enough of them to fill the chip at 256 threads a workgroup: C5's
  // 123 K groups 41.6 -> 39.8 us (both launches); C2's 18 K groups ran 0.5 us
  // slower (72 workgroups), also at 64 threads a workgroup, and keep one each.
  const bool v4 = (NC * FD) % 4 == 0 && NC * FD >= 4 * 65536 && (reinterpret_cast<uintptr_t>(a.work) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(a.g_phi) & 7) == 0;
  if (v4)
    hipLaunchKernelGGL(weights_reduce_kernel<true>, dim3((unsigned)((NC * FD / 4 + 255) / 256 + 1)), dim3(256), 0,
                       s, a, R);
  else
    hipLaunchKernelGGL(weights_reduce_kernel<false>, dim3((unsigned)(qb + 1)), dim3(256), 0, s, a, R);
  return hipGetLastError();
}

// ------------------------------------------------------- Sinkhorn backward
// One 256-thread workgroup holds 256 / n^2 matrices, one element per thread.
// Forward T[0] = P + eps, T[1] = T[0] / (colsum + eps), then row / column
// steps; backward through y = x / (sum(x) + eps):  g_x = (g_y - sum(g_y * y)) / (sum(x) + eps),
// and through the softmax: g_m = P * (g - rowsum(g * P)).
// The trajectory is not kept whole: the forward stores every K-th iterate
// (checkpoints), and the backward walks the segments from the last, first
// recomputing a segment's K + 1 iterates from its checkpoint with the same
// operations (so the same bits).  LDS holds the softmax P, J checkpoints, one
// segment and a scratch row: (J + K + 3) * 1 KiB with K ~ J ~ sqrt(steps).
__global__ __launch_bounds__(256) void sinkhorn_bwd_kernel(const void* __restrict__ m_in, int in_dt,
                                                           const void* __restrict__ g_out, int g_dt,
                                                           void* __restrict__ g_in, int gi_dt,
                                                           int64_t batch, int n, int iters, float eps,
                                                           int K) {
  extern __shared__ float lds[];
  const int G = n * n;
  const int per = 256 / G;                  // matrices per workgroup
  const int tid = threadIdx.x;
  const int m_loc = tid / G;
  const int e = tid - m_loc * G;
  const int r = e / n;
  const int c = e - r * n;
  const int64_t mat = (int64_t)blockIdx.x * per + m_loc;
  const bool live = m_loc < per && mat < batch;
  const int64_t idx = mat * G + e;
  const int steps = 2 * (iters > 1 ? iters : 1);
  const int J = (steps - 1 + K - 1) / K;    // segments of backward steps 1 .. steps - 1
  float* P = lds;                           // [256]
  float* CK = lds + 256;                    // [J][256] iterate jK
  float* SEG = CK + (int64_t)J * 256;       // [K + 1][256] iterates jK .. jK + K
  float* S = SEG + (int64_t)(K + 1) * 256;  // [256] scratch
  // First element of this row / column (stride n).  Threads past the last
  // whole matrix (256 % n^2 of them) read matrix 0 and store nothing.
  const int rb = m_loc < per ? tid - e + r * n : 0;
  const int cb = m_loc < per ? tid - e + c : 0;
  auto row_sum = [&](const float* A) {
    float s = 0.f;
    for (int j = 0; j < n; ++j) s += A[rb + j];
    return s;
  };
  auto col_sum = [&](const float* A) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s += A[cb + i * n];
    return s;
  };
  // One forward step s (odd: column, even: row) from X into Y.
  auto fwd_step = [&](int s, const float* X, float* Y) {
    const float den = ((s & 1) ? col_sum(X) : row_sum(X)) + eps;
    Y[tid] = X[tid] / den;
  };

  // forward recompute, keeping iterates 0, K, 2K, ... (two SEG rows alternate)
  // both inputs' loads issue before either is waited for
  const uint32_t mb = live ? ld_raw(m_in, idx, in_dt) : 0u;
  const uint32_t gb = live ? ld_raw(g_out, idx, g_dt) : 0u;
  const float v = raw_to_f32(mb, in_dt);
  S[tid] = v;
  __syncthreads();
  float mx = -INFINITY;
  for (int j = 0; j < n; ++j) mx = fmaxf(mx, S[rb + j]);
  const float ex = expf(v - mx);
  __syncthreads();
  S[tid] = ex;
  __syncthreads();
  const float p = ex / row_sum(S);
  P[tid] = p;
  SEG[tid] = p + eps;
  CK[tid] = p + eps;
  __syncthreads();
  for (int s = 1; s < (J - 1) * K + 1; ++s) {  // up to the last checkpoint
    const float* X = SEG + (int64_t)((s - 1) & 1) * 256;
    float* Y = SEG + (int64_t)(s & 1) * 256;
    fwd_step(s, X, Y);
    if (s % K == 0) CK[(int64_t)(s / K) * 256 + tid] = Y[tid];
    __syncthreads();
  }
  // backward, one segment at a time from the last
  float g = raw_to_f32(gb, g_dt);
  for (int j = J - 1; j >= 0; --j) {
    const int s0 = j * K;
    const int s1 = s0 + K < steps - 1 ? s0 + K : steps - 1;  // last backward step of the segment
    __syncthreads();                      // every read of the previous segment done
    SEG[tid] = CK[(int64_t)j * 256 + tid];
    __syncthreads();
    for (int s = s0 + 1; s <= s1; ++s) {
      fwd_step(s, SEG + (int64_t)(s - 1 - s0) * 256, SEG + (int64_t)(s - s0) * 256);
      __syncthreads();
    }
    for (int s = s1; s >= s0 + 1; --s) {
      const float* X = SEG + (int64_t)(s - 1 - s0) * 256;
      const float* Y = SEG + (int64_t)(s - s0) * 256;
      __syncthreads();
      S[tid] = g * Y[tid];
      __syncthreads();
      const bool col = s & 1;
      const float dot = col ? col_sum(S) : row_sum(S);
      const float den = (col ? col_sum(X) : row_sum(X)) + eps;
      g = (g - dot) / den;
    }
  }
  __syncthreads();
  S[tid] = g * p;
  __syncthreads();
  const float gm = p * (g - row_sum(S));
  if (live) st_any(g_in, idx, gi_dt, gm);
}

// n in {2, 4, 8}: one wave per workgroup, one matrix element per lane
// (64 / n^2 matrices per wave), row and column sums as DPP / permlane
// butterflies inside the matrix's lanes (row_reduce / col_sum).  Each lane
// keeps its own forward trajectory in private LDS slots (the iterate after
// each step and that step's divisor), so no barrier is needed; divisions are
// reciprocal * multiply, as in the forward kernels.
template <int N>
__global__ __launch_bounds__(64) void sinkhorn_bwd_lanes_kernel(const void* __restrict__ m_in, int in_dt,
                                                                const void* __restrict__ g_out, int g_dt,
                                                                void* __restrict__ g_in, int gi_dt,
                                                                int64_t batch, int iters, float eps) {
  extern __shared__ float lds[];
  constexpr int G = N * N;
  const int lane = threadIdx.x;
  const int64_t idx = (int64_t)blockIdx.x * 64 + lane;  // element index (64 / G matrices per wave)
  const bool live = idx < batch * G;
  const int steps = 2 * (iters > 1 ? iters : 1);
  float* Y = lds;                 // [steps][64] iterate after step s
  float* D = lds + steps * 64;    // [steps][64] divisor of step s (1 for the softmax step)

  // both inputs' loads issue before either is waited for
  const uint32_t mb = live ? ld_raw(m_in, idx, in_dt) : 0u;
  const uint32_t gb = live ? ld_raw(g_out, idx, g_dt) : 0u;
  const float v = raw_to_f32(mb, in_dt);
  const float mx = row_reduce<N, OpMax>(v);
  const float ex = expf(v - mx);
  const float p = ex * __builtin_amdgcn_rcpf(row_reduce<N, OpAdd>(ex));
  float t = p + eps;
  Y[lane] = t;
  for (int st = 1; st < steps; ++st) {  // odd: column step, even: row step
    const float den = ((st & 1) ? col_sum<N>(t) : row_reduce<N, OpAdd>(t)) + eps;
    t = t * __builtin_amdgcn_rcpf(den);
    Y[st * 64 + lane] = t;
    D[st * 64 + lane] = den;
  }
  float gr = raw_to_f32(gb, g_dt);
  for (int st = steps - 1; st >= 1; --st) {
    const float y = Y[st * 64 + lane];
    const float gy = gr * y;
    const float dot = (st & 1) ? col_sum<N>(gy) : row_reduce<N, OpAdd>(gy);
    gr = (gr - dot) * __builtin_amdgcn_rcpf(D[st * 64 + lane]);
  }
  const float gm = p * (gr - row_reduce<N, OpAdd>(gr * p));
  if (live) st_any(g_in, idx, gi_dt, gm);
}

// The same recurrence with the trajectory in registers, for schedules of at
// most MAXS steps (2 * iters): no LDS, so occupancy is set by registers alone
// and every access is a register read.  The steps run fully unrolled behind a
// uniform bound on the real step count.  (The reference's 20 iterations take
// the 2 x 2-block kernel above at n in {2, 4, 8}.)
template <int N, int MAXS>
__global__ __launch_bounds__(256) void sinkhorn_bwd_regs_kernel(const void* __restrict__ m_in, int in_dt,
                                                                const void* __restrict__ g_out, int g_dt,
                                                                void* __restrict__ g_in, int gi_dt,
                                                                int64_t batch, int iters, float eps) {
  constexpr int G = N * N;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // element index
  const bool live = idx < batch * G;
  const int steps = 2 * (iters > 1 ? iters : 1);
  float Y[MAXS];
  float R[MAXS];  // 1 / divisor of each step
  // Both inputs' elements load together, as the 4-byte words that hold them
  // (descriptors of the exact sizes; n^2 is even, so a 16-bit element's word
  // lies inside its tensor): the per-dtype branches of ld_any made each load
  // wait for the one before it.
  const int es_m = in_dt == kF32 ? 4 : 2, es_g = g_dt == kF32 ? 4 : 2;
  const uint32_t mw = buf_load4z(make_rsrc(m_in, (uint32_t)(batch * G * es_m)), live ? word_off(idx, in_dt) : kBufOob).v[0];
  const uint32_t gw = buf_load4z(make_rsrc(g_out, (uint32_t)(batch * G * es_g)), live ? word_off(idx, g_dt) : kBufOob).v[0];
  const float v = word_elem(mw, idx, in_dt);
  const float mx = row_reduce<N, OpMax>(v);
  const float ex = expf(v - mx);
  const float p = ex * __builtin_amdgcn_rcpf(row_reduce<N, OpAdd>(ex));
  float t = p + eps;
  Y[0] = t;
  R[0] = 1.f;
#pragma unroll
  for (int st = 1; st < MAXS; ++st) {  // odd: column step, even: row step
    if (st < steps) {                  // uniform
      const float den = ((st & 1) ? col_sum<N>(t) : row_reduce<N, OpAdd>(t)) + eps;
      R[st] = __builtin_amdgcn_rcpf(den);
      t = t * R[st];
      Y[st] = t;
    }
  }
  float gr = word_elem(gw, idx, g_dt);
#pragma unroll
  for (int st = MAXS - 1; st >= 1; --st) {
    if (st < steps) {
      const float gy = gr * Y[st];
      const float dot = (st & 1) ? col_sum<N>(gy) : row_reduce<N, OpAdd>(gy);
      gr = (gr - dot) * R[st];
    }
  }
  const float gm = p * (gr - row_reduce<N, OpAdd>(gr * p));
  if (live) st_any(g_in, idx, gi_dt, gm);
}

// 2 x 2 blocks per lane: one n x n matrix per (n/2)^2 lanes (n = 8: 16 lanes,
// a DPP row; n = 4: a quad; n = 2: one lane), lane j holding rows
// 2 (j / (n/2)) .. + 1 and columns 2 (j % (n/2)) .. + 1.  A row sum is one
// in-lane add and row_reduce<n/2> (lane xor 1, 2); a column sum one in-lane
// add and col_sum<n/2> (n = 8: lanes j + 4, 8, 12 by two rotations; n = 4:
// lane xor 2), so both steps cost the same.  At n = 8 this replaced the
// half-row layout of the forward's sk8_* Sinkhorn (lane j: row j & 7, columns
// 4 (j >> 3) .. + 3), whose column step took a 3-stage butterfly for each of
// four columns and DPP broadcasts of the reciprocals: 1690 -> 1429 VALU
// instructions a wave, C5 shape (8192 matrices) 8.1-8.2 -> 6.9-7.0 us; at
// n = 4 it replaced one element a lane (531 VALU instructions a wave for 4
// matrices, 1263 now for 16), C2 shape (16384 matrices) 6.0-6.4 -> 4.8-4.9
// us, though the grid now fills one wave a SIMD.  Each lane keeps its two
// rows' and two columns' reciprocals of every step (~244 VGPRs).  The trajectory: the iterate after each column step (4 values) and
// both reciprocals; the iterate after a row step is recomputed from the
// column iterate before it with the forward's own multiply.
template <int N, int K>
__global__ __launch_bounds__(256) void sinkhorn_bwd_b22_kernel(const void* __restrict__ m_in, int in_dt,
                                                               const void* __restrict__ g_out, int g_dt,
                                                               void* __restrict__ g_in, int gi_dt,
                                                               int64_t batch, float eps) {
  static_assert(N == 2 || N == 4 || N == 8, "2 x 2 blocks: n in {2, 4, 8}");
  constexpr int H = N / 2;                                             // blocks a row
  constexpr int L = H * H;                                             // lanes a matrix
  const int64_t mi = ((int64_t)blockIdx.x * 256 + threadIdx.x) / L;  // matrix
  const int j = threadIdx.x % L;
  const bool live = mi < batch;
  // element (a, b) of this lane's block: row 2 (j / H) + a, column 2 (j % H) + b
  const int64_t e0 = mi * N * N + (j / H) * 2 * N + (j % H) * 2;  // (0, 0); (1, 0) is N further
  // Both inputs' two row pairs, one 8-byte buffer load each, issued together
  // (a 16-bit input's pair is the first half of its 8 bytes); the descriptors
  // hold the exact sizes, so bytes past the end read zero.
  const int es_m = in_dt == kF32 ? 4 : 2, es_g = g_dt == kF32 ? 4 : 2;
  const auto rm = make_rsrc(m_in, (uint32_t)(batch * N * N * es_m));
  const auto rg = make_rsrc(g_out, (uint32_t)(batch * N * N * es_g));
  U32x4 mw[2], gw[2];
#pragma unroll
  for (int a = 0; a < 2; ++a) mw[a] = buf_load8z(rm, live ? (uint32_t)(e0 + N * a) * es_m : kBufOob);
#pragma unroll
  for (int a = 0; a < 2; ++a) gw[a] = buf_load8z(rg, live ? (uint32_t)(e0 + N * a) * es_g : kBufOob);
  float t[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) t[a][b] = word4_elem(mw[a], b, in_dt);
  // softmax over each row, + eps
  float p[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const float mx = row_reduce<H, OpMax>(fmaxf(t[a][0], t[a][1]));
    p[a][0] = expf(t[a][0] - mx);
    p[a][1] = expf(t[a][1] - mx);
    const float rs = __builtin_amdgcn_rcpf(row_reduce<H, OpAdd>(p[a][0] + p[a][1]));
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      p[a][b] = mul_nc(p[a][b], rs);
      t[a][b] = p[a][b] + eps;
    }
  }
  float Y[K][2][2];  // iterate after column step k
  float RC[K][2];    // column step k: reciprocals of this lane's two columns
  float RR[K][2];    // row step k (before column step k, k >= 1): of its two rows
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (k > 0) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        RR[k][a] = __builtin_amdgcn_rcpf(row_reduce<H, OpAdd>(t[a][0] + t[a][1]) + eps);
        t[a][0] = mul_nc(t[a][0], RR[k][a]);
        t[a][1] = mul_nc(t[a][1], RR[k][a]);
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      RC[k][b] = __builtin_amdgcn_rcpf(col_sum<H>(t[0][b] + t[1][b]) + eps);
      t[0][b] = mul_nc(t[0][b], RC[k][b]);
      t[1][b] = mul_nc(t[1][b], RC[k][b]);
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) Y[k][a][b] = t[a][b];
  }
  float gr[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) gr[a][b] = word4_elem(gw[a], b, g_dt);
#pragma unroll
  for (int k = K - 1; k >= 0; --k) {
    // column step k: y = Y[k]
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const float d = col_sum<H>(mul_nc(gr[0][b], Y[k][0][b]) + mul_nc(gr[1][b], Y[k][1][b]));
      gr[0][b] = (gr[0][b] - d) * RC[k][b];
      gr[1][b] = (gr[1][b] - d) * RC[k][b];
    }
    if (k > 0) {  // row step k: y = Y[k - 1] * RR[k], as the forward formed it
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const float d = row_reduce<H, OpAdd>(mul_nc(gr[a][0], mul_nc(Y[k - 1][a][0], RR[k][a])) +
                                             mul_nc(gr[a][1], mul_nc(Y[k - 1][a][1], RR[k][a])));
        gr[a][0] = (gr[a][0] - d) * RR[k][a];
        gr[a][1] = (gr[a][1] - d) * RR[k][a];
      }
    }
  }
  // softmax: t0 = p + eps, so the gradient of p is gr
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const float dp = row_reduce<H, OpAdd>(mul_nc(gr[a][0], p[a][0]) + mul_nc(gr[a][1], p[a][1]));
    if (live) {
#pragma unroll
      for (int b = 0; b < 2; ++b) st_any(g_in, e0 + N * a + b, gi_dt, p[a][b] * (gr[a][b] - dp));
    }
  }
}

// Segment length K of sinkhorn_bwd_kernel for a schedule of 2 * iters steps
// (about the square root of the step count) and its LDS bytes.
int sinkhorn_bwd_segment(int iters) {
  const int steps = 2 * (iters > 1 ? iters : 1);
  int K = 1;
  while (K * K < steps - 1) ++K;
  return K;
}
size_t sinkhorn_bwd_lds_bytes(int iters) {
  const int steps = 2 * (iters > 1 ? iters : 1);
  const int K = sinkhorn_bwd_segment(iters);
  const int J = (steps - 1 + K - 1) / K;
  return (size_t)(J + K + 3) * 256 * sizeof(float);
}

hipError_t launch_sinkhorn_bwd(const void* m_in, int in_dtype, const void* g_out, int g_dtype,
                               void* g_in, int gi_dtype, int64_t batch, int n, int iters,
                               float eps, hipStream_t s) {
  // The register kernels read both inputs through buffer descriptors: 32-bit
  // byte offsets, 4-byte aligned bases.  Anything else takes the kernels below.
  const bool buf_ok = batch * n * n * 4 < (int64_t)kBufOob && ((uintptr_t)m_in & 3) == 0 &&
                      ((uintptr_t)g_out & 3) == 0;
  // The 2 x 2-block kernel at the two schedules in use: 20 iterations (the
  // models' configs) and 10 (MHCConnection_Fused's default).
  if (buf_ok && (n == 2 || n == 4 || n == 8) && (iters == 20 || iters == 10)) {
    const int64_t blocks = (batch * (n / 2) * (n / 2) + 255) / 256;  // (n/2)^2 lanes a matrix
#define MHC_SK_B22(NN, KK)                                                                      \
  hipLaunchKernelGGL((sinkhorn_bwd_b22_kernel<NN, KK>), dim3((unsigned)blocks), dim3(256), 0, s, \
                     m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, eps)
    if (iters == 20) {
      if (n == 2) MHC_SK_B22(2, 20); else if (n == 4) MHC_SK_B22(4, 20); else MHC_SK_B22(8, 20);
    } else {
      if (n == 2) MHC_SK_B22(2, 10); else if (n == 4) MHC_SK_B22(4, 10); else MHC_SK_B22(8, 10);
    }
#undef MHC_SK_B22
    return hipGetLastError();
  }
  if (buf_ok && (n == 2 || n == 4 || n == 8) && iters <= 20) {
    const int64_t blocks = (batch * n * n + 255) / 256;
    switch (n) {
      case 2: hipLaunchKernelGGL((sinkhorn_bwd_regs_kernel<2, 40>), dim3((unsigned)blocks), dim3(256), 0, s, m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, iters, eps); break;
      case 4: hipLaunchKernelGGL((sinkhorn_bwd_regs_kernel<4, 40>), dim3((unsigned)blocks), dim3(256), 0, s, m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, iters, eps); break;
      default: hipLaunchKernelGGL((sinkhorn_bwd_regs_kernel<8, 40>), dim3((unsigned)blocks), dim3(256), 0, s, m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, iters, eps); break;
    }
    return hipGetLastError();
  }
  if ((n == 2 || n == 4 || n == 8) && iters <= kSinkhornBwdLanesMaxIters) {
    const int steps = 2 * (iters > 1 ? iters : 1);
    const size_t lds = (size_t)2 * steps * 64 * sizeof(float);
    const int64_t blocks = (batch * n * n + 63) / 64;
    switch (n) {
      case 2: hipLaunchKernelGGL(sinkhorn_bwd_lanes_kernel<2>, dim3((unsigned)blocks), dim3(64), lds, s, m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, iters, eps); break;
      case 4: hipLaunchKernelGGL(sinkhorn_bwd_lanes_kernel<4>, dim3((unsigned)blocks), dim3(64), lds, s, m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, iters, eps); break;
      default: hipLaunchKernelGGL(sinkhorn_bwd_lanes_kernel<8>, dim3((unsigned)blocks), dim3(64), lds, s, m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, iters, eps); break;
    }
    return hipGetLastError();
  }
  const int G = n * n;
  const int per = 256 / G;
  const int64_t blocks = (batch + per - 1) / per;
  const int K = sinkhorn_bwd_segment(iters);
  const size_t lds = sinkhorn_bwd_lds_bytes(iters);
  hipLaunchKernelGGL(sinkhorn_bwd_kernel, dim3((unsigned)blocks), dim3(256), lds, s, m_in, in_dtype,
                     g_out, g_dtype, g_in, gi_dtype, batch, n, iters, eps, K);
  return hipGetLastError();
}

}  // namespace mhc
