/*
 * mhc_amd.h -- C ABI of the MI355X (gfx950) mHC forward and backward kernels.
 *
 * Every entry point takes raw device pointers, plain sizes and a hipStream_t,
 * enqueues its kernels on that stream and returns without synchronising.
 * The caller allocates every output (as the reference's autograd Functions do
 * with torch.empty); the library never allocates or frees device memory.  It
 * keeps no per-call state, so calls are re-entrant and capturable, with one
 * exception below.  It has three process-wide settings, all kernel choices:
 * mhc_pre_token_threshold, mhc_pre_group_split_tokens and
 * mhc_pre_row_staging.  One entry point
 * (mhc_pre_bwd_weights) needs scratch for token-range partial sums; the caller
 * passes it as a workspace argument, or calls mhc_pre_bwd_weights_noalloc,
 * which uses a 32 MiB static device array the library holds per device
 * instead.  That array is the exception: calls of the noalloc entry point
 * that overlap on one device share it and race.
 *
 * Return value: 0 on success.  Otherwise a hipError_t code
 * (hipErrorInvalidValue = 1 for bad arguments); mhc_last_error() then returns a
 * message for the calling thread.
 *
 * Tensors are contiguous, row-major.  Shapes below use M = B*L tokens, n
 * streams, C = hidden size, FD = width of the fused projection:
 *   FD = 2n + n*n (full mHC), 2n (no H_res), n (MHCHead).
 * Scalars and biases (alpha_*, bias_*) are device pointers, never host
 * floats, so no call needs a device-to-host sync.
 *
 * Reference paths cited as file:line are relative to the minimind-mhc
 * repository root.
 */
#ifndef MHC_AMD_H_
#define MHC_AMD_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage dtype tags. */
#define MHC_DTYPE_F32 0
#define MHC_DTYPE_BF16 1
#define MHC_DTYPE_F16 2

/* Projection layouts for mhc_phi_pack / mhc_phi_packed_bytes. */
#define MHC_MODE_FULL 0   /* phi [n*C, 2n+n*n]: MHCConnection_Fused        */
#define MHC_MODE_NOHRES 1 /* phi [n*C, 2n]:     MHCConnection_FusedNoHres  */
#define MHC_MODE_HEAD 2   /* phi [n*C, n]:      MHCHead                    */
#define MHC_MODE_RMS 3    /* no phi:            MHCHead with n == 1 (RMSNorm), backward only */

/* ABI revision (bumped on any signature change). */
int mhc_abi_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* mhc_last_error(void);

/*
 * One-time set-up for every visible device: looks up each device's copy of
 * the scratch array that mhc_pre_bwd_weights_noalloc uses.  Call it once
 * before capturing that entry point in a HIP graph; the entry point refuses a
 * device it has not seen while its stream is being captured.  Idempotent,
 * thread-safe, no device allocation.
 * No reference counterpart (the reference has no allocation-free path).
 */
int mhc_init(void);

/*
 * Size in bytes of the MFMA operand image of phi for (n, C, mode), or 0 when
 * that shape has no MFMA kernel (n not in {1,2,4,8,16}, C % 8 != 0, n == 1
 * with C > 1024, MHCHead with n == 1, or an image past 2 GiB).  Host-only, no
 * device work.
 * No reference counterpart: the reference re-reads phi row-major per token
 * (model/mhc_fused.py:217-229); this build re-lays it out once per weight
 * version for MFMA B-operand loads.
 */
int64_t mhc_phi_packed_bytes(int n, int C, int mode);

/*
 * Write the MFMA operand image of phi [n*C, FD] (bf16) into packed
 * (mhc_phi_packed_bytes bytes).  phi_dtype must be MHC_DTYPE_BF16.
 * No reference counterpart (see mhc_phi_packed_bytes).
 */
int mhc_phi_pack(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                 hipStream_t stream);

/*
 * Size in bytes of the split-operand image of an fp32 phi for (n, C, mode), or
 * 0 when that shape has no fp32 MFMA kernel.  Shapes with one: n in {1,2,4}
 * with C <= 1024 (16-column tiles of hi | lo pairs, one-workgroup-per-tile
 * kernel), n == 8 at any C and n in {2,4} with C > 1024 (the bf16 K-streamed
 * image twice, hi then lo); C % 8 == 0 and not MHCHead with n == 1 for all.
 * n == 16 has none.  Host-only, no device work.
 * No reference counterpart: the reference's fused kernel computes the fp32
 * projection elementwise (model/mhc_fused.py:217-230); this build runs it as
 * bf16 MFMAs on hi / lo splits of both operands.
 */
int64_t mhc_phi_split_bytes(int n, int C, int mode);

/*
 * Write the split-operand image of phi [n*C, FD] (any dtype; each value is
 * split into bf16(v) and bf16(v - bf16(v))) into packed (mhc_phi_split_bytes
 * bytes).  No reference counterpart (see mhc_phi_split_bytes).
 */
int mhc_phi_pack_split(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                       hipStream_t stream);

/*
 * Full mHC pre phase fused with Sinkhorn: RMS over the n*C row (no gain),
 * projection x_norm @ phi, gates, Sinkhorn-Knopp of H_res, and the
 * pre-aggregate sublayer_in = sum_i h_pre[i] * x[i].
 *
 * Replaces, in one launch:
 *   _PrePhaseFullFn.forward        model/mhc_fused.py:575-641
 *   (its kernel                    model/mhc_fused.py:163-268)
 *   sinkhorn_normalize(h_res_raw)  model/mhc_fused.py:140-154, called at :828-830
 *
 *   x            [M, n*C]   x_dtype (f32 / bf16 / f16)
 *   phi          [n*C, FD]  phi_dtype, FD = 2n + n*n, columns [pre | post | res]
 *   phi_packed   image of phi for the MFMA kernels, or NULL (then a VALU kernel
 *                runs): the mhc_phi_pack image for bf16 x and bf16 phi, the
 *                mhc_phi_pack_split image for fp32 x and fp32 phi; ignored for
 *                other dtype pairs
 *   alpha_pre/post/res  0-dim scalars, bias_pre/post [n], bias_res [n, n];
 *                all param_dtype
 *   sublayer_in  [M, C]     x_dtype               (required)
 *   h_pre        [M, n]     x_dtype               (optional, NULL to skip)
 *   h_post       [M, n]     x_dtype               (required)
 *   h_res_raw    [M, n, n]  x_dtype, pre-Sinkhorn (optional)
 *   h_res        [M, n, n]  x_dtype, Sinkhorn output (NULL: Sinkhorn skipped)
 *   inv_rms      [M]        fp32                  (optional)
 *   mixes_raw    [M, FD]    fp32                  (optional)
 *   sinkhorn_iters: reference count (1 softmax-row pass + iters column passes,
 *                   iters - 1 extra row passes); <= 1 behaves as 1.
 *   x_ssq        [M, C / 128] fp32 or NULL: per-row partial sums of squares
 *                of x as mhc_post_fwd / mhc_expand_norm_fwd write them
 *                (out_ssq), row t's sum of squares = sum_j x_ssq[t][j] in j
 *                order.  bf16 x with C % 128 == 0 only.  Used where the
 *                kernel would otherwise read x once more to form the sums
 *                (n = 8, n = 16, or C > 1024), ignored elsewhere; inv_rms
 *                then comes from these sums (equal to rounding).  No
 *                reference counterpart.
 */
int mhc_pre_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype, const void* phi_packed,
                const void* alpha_pre, const void* bias_pre, const void* alpha_post,
                const void* bias_post, const void* alpha_res, const void* bias_res,
                int param_dtype, void* sublayer_in, void* h_pre, void* h_post, void* h_res_raw,
                void* h_res, float* inv_rms, float* mixes_raw, int64_t M, int n, int C,
                float post_mult, float pre_eps, float rms_eps, int sinkhorn_iters,
                float sinkhorn_eps, const float* x_ssq, hipStream_t stream);

/*
 * mHC pre phase without H_res (use_mhc = 2): FD = 2n, no Sinkhorn.
 * Replaces _PrePhaseFn.forward  model/mhc_fused_no_hres.py:400-463
 *          (its kernel          model/mhc_fused_no_hres.py:48-145).
 * Arguments as mhc_pre_fwd without the res segment.
 */
int mhc_pre_nohres_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                       const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                       const void* alpha_post, const void* bias_post, int param_dtype,
                       void* sublayer_in, void* h_pre, void* h_post, float* inv_rms,
                       float* mixes_raw, int64_t M, int n, int C, float post_mult, float pre_eps,
                       float rms_eps, const float* x_ssq, hipStream_t stream);

/*
 * Post phase: out[t,i,:] = sum_j h_res[t,i,j] * x[t,j,:] + h_post[t,i] * f_out[t,:].
 * Replaces _PostPhaseFullFn.forward  model/mhc_fused.py:720-744
 *          (its kernel               model/mhc_fused.py:416-459).
 *   x [M, n*C] x_dtype; h_res [M, n, n] and h_post [M, n] h_dtype;
 *   f_out [M, C] f_dtype; out [M, n*C] x_dtype (must not alias x).
 *   out_ssq [M, C / 128] fp32 or NULL: per-row partial sums of the squares
 *   of out (as stored), for the next pre launch's x_ssq (bf16 x, gates and
 *   F, C % 128 == 0, 16-byte aligned tensors; no reference counterpart).
 */
int mhc_post_fwd(const void* x, int x_dtype, const void* h_res, const void* h_post, int h_dtype,
                 const void* f_out, int f_dtype, void* out, int64_t M, int n, int C,
                 float* out_ssq, hipStream_t stream);

/*
 * Post phase without H_res: out = x + h_post (x) f_out.
 * Replaces _PostPhaseFn.forward  model/mhc_fused_no_hres.py:535-556
 *          (its kernel           model/mhc_fused_no_hres.py:284-316).
 */
int mhc_post_nohres_fwd(const void* x, int x_dtype, const void* h_post, int h_dtype,
                        const void* f_out, int f_dtype, void* out, int64_t M, int n, int C,
                        float* out_ssq, hipStream_t stream);

/*
 * MHCHead exit: out = sum_i (sigmoid(alpha * (x_norm @ phi)_i + bias_i) + pre_eps) * x_i,
 * phi [n*C, n], alpha shape (1,), bias [n].  For n == 1 it is the plain
 * RMSNorm out = x * inv_rms (phi, alpha, bias ignored and may be NULL).
 * Replaces _MHCHeadFn.forward     model/mhc_common.py:315-357
 *          (its kernel            model/mhc_common.py:128-195)
 *          and MHCHead.forward's n == 1 branch  model/mhc_common.py:438-442.
 *   out [M, C] x_dtype; inv_rms [M], mix_raw [M, n] fp32 optional;
 *   x_ssq as mhc_pre_fwd.
 */
int mhc_head_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                 const void* phi_packed, const void* alpha, const void* bias, int param_dtype,
                 void* out, float* inv_rms, float* mix_raw, int64_t M, int n, int C, float pre_eps,
                 float rms_eps, const float* x_ssq, hipStream_t stream);

/*
 * Batched Sinkhorn-Knopp of [batch, n, n] matrices, fp32 arithmetic, output
 * in the input dtype; n <= 32 (any n, fastest for n in {1,2,4,8}).
 * Replaces _SinkhornFn.forward  model/mhc_fused.py:111-128
 *          (its kernel          model/mhc_fused.py:61-93).
 */
int mhc_sinkhorn_fwd(const void* m_in, void* m_out, int dtype, int64_t batch, int n, int iters,
                     float eps, hipStream_t stream);

/*
 * StreamExpand: out[t, i*C + c] = x[t, c] for i < n (elem_bytes 2 or 4).
 * Replaces StreamExpand.forward  model/mhc_common.py:115-119.
 */
int mhc_stream_expand_fwd(const void* x, void* out, int elem_bytes, int64_t M, int n, int C,
                          hipStream_t stream);

/* --------------------------------------------------- fused input norms
 * The model wraps every sublayer as F(z) = sublayer(RMSNorm_C(z)) and ends
 * with RMSNorm_C(MHCHead(x)) (model/model_minimind.py:326-336, :367-370).  The
 * *_norm_fwd variants apply that RMSNorm (gain norm_weight [C] of norm_dtype,
 * eps norm_eps) to the main output inside the same launch:
 *   out = round(s * (1 / sqrt(mean_c(s^2) + norm_eps)) * norm_weight)
 * where s is the pre-aggregate (head output) rounded to x_dtype, i.e. the
 * tensor the reference's nn.RMSNorm receives.  All other outputs are those
 * of the plain entry point.  Forward only: training keeps the separate norm,
 * whose backward needs the un-normed s.
 */

/*
 * mhc_pre_fwd + the sublayer's input RMSNorm.
 * Replaces _PrePhaseFullFn.forward   model/mhc_fused.py:575-641
 *          + self.attn_in_norm / self.ffn_in_norm applied to its output
 *            inside F                model/model_minimind.py:330, :336.
 */
int mhc_pre_norm_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                     const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                     const void* alpha_post, const void* bias_post, const void* alpha_res,
                     const void* bias_res, int param_dtype, void* sublayer_in_normed, void* h_pre,
                     void* h_post, void* h_res_raw, void* h_res, float* inv_rms,
                     float* mixes_raw, int64_t M, int n, int C, float post_mult, float pre_eps,
                     float rms_eps, int sinkhorn_iters, float sinkhorn_eps,
                     const void* norm_weight, int norm_dtype, float norm_eps, const float* x_ssq,
                     hipStream_t stream);

/*
 * mhc_pre_nohres_fwd + the sublayer's input RMSNorm.
 * Replaces _PrePhaseFn.forward  model/mhc_fused_no_hres.py:400-463
 *          + the in-F norm      model/model_minimind.py:330, :336.
 */
int mhc_pre_nohres_norm_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                            const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                            const void* alpha_post, const void* bias_post, int param_dtype,
                            void* sublayer_in_normed, void* h_pre, void* h_post, float* inv_rms,
                            float* mixes_raw, int64_t M, int n, int C, float post_mult,
                            float pre_eps, float rms_eps, const void* norm_weight, int norm_dtype,
                            float norm_eps, const float* x_ssq, hipStream_t stream);

/*
 * mhc_head_fwd + the model's final RMSNorm.
 * Replaces self.norm = Sequential(MHCHead, RMSNorm)  model/model_minimind.py:367-370
 *          (MHCHead.forward model/mhc_common.py:435-450).
 */
int mhc_head_norm_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                      const void* phi_packed, const void* alpha, const void* bias, int param_dtype,
                      void* out_normed, float* inv_rms, float* mix_raw, int64_t M, int n, int C,
                      float pre_eps, float rms_eps, const void* norm_weight, int norm_dtype,
                      float norm_eps, const float* x_ssq, hipStream_t stream);

/*
 * The model's entry: RMSNorm over C with gain norm_weight, then n copies:
 *   out[t, i*C + c] = round(x[t, c] * (1 / sqrt(mean_c(x[t]^2) + eps)) * w[c]).
 * Replaces self.embed_up_norm = Sequential(RMSNorm, StreamExpand)
 *          model/model_minimind.py:365, applied at :385
 *          (StreamExpand.forward model/mhc_common.py:115-119).
 *   x [M, C] x_dtype; out [M, n*C] x_dtype; out_ssq [M, C / 128] fp32 or
 *   NULL: the written row's sum of squares in out_ssq[t][0], the other
 *   partials zero (the next pre launch's x_ssq; bf16, C % 128 == 0).
 */
int mhc_expand_norm_fwd(const void* x, int x_dtype, const void* norm_weight, int norm_dtype,
                        void* out, int64_t M, int n, int C, float eps, float* out_ssq,
                        hipStream_t stream);

/*
 * Batch size (tokens) at or below which the pre-phase entry points run the
 * small-batch kernel (one workgroup per group of up to 16 tokens, phi read
 * from L2) instead of the large-batch ones (bf16, packed phi, n in {1, 2, 4,
 * 8}, C <= 1024; n = 16 and wider rows take the K-streamed kernel at every
 * size; default 1024); max_tokens < 0 only queries.  Both sides give
 * bit-identical results.  Returns the previous value.  Process-wide setting,
 * not synchronised with calls in flight.
 * No reference counterpart (the reference launches one program per token at
 * every size, model/mhc_fused.py:615-641).
 */
int64_t mhc_pre_token_threshold(int64_t max_tokens);

/*
 * Whether the persistent pre kernel loads x tiles as whole rows and stages
 * them through LDS (C a multiple of 256, phi resident in registers, no fused
 * norm; on by default) rather than loading the MFMA operand layout directly.
 * The row-staged kernel sums each row's squares in row order, so inv_rms may
 * differ in its last bit from the operand-layout kernel's and, through
 * x_norm's bf16 rounding, a token's gates by a rounding step (rounding-level
 * agreement; tokens whose mixes agree match bit for bit).  The small-batch
 * kernel sums in whichever order the persistent kernel would use, so the
 * token threshold stays bit-identical under either setting.  The row loads
 * stream faster on MI355X.
 * on < 0 only queries; returns the previous setting (0 or 1).  Process-wide,
 * not synchronised with calls in flight.  No reference counterpart (a
 * scheduling choice of this implementation).
 */
int mhc_pre_row_staging(int on);

/*
 * Batch size (tokens) at or below which the n = 8 small-batch pre phase (bf16,
 * packed phi, 4 * FD <= 2 * C) runs as two launches: the projection with each
 * group's 16-column output tiles on workgroups of their own (each reads 1 / NT
 * of phi instead of all of it), the finished mixes parked as fp32 in the
 * sublayer-input rows, then the gates, Sinkhorn, pre-aggregate and norm.  The
 * same MFMA chains and sums as the one-launch kernel: bit-identical results.
 * Default 128; max_tokens < 0 only queries; returns the previous value.
 * Process-wide, not synchronised with calls in flight.  No reference
 * counterpart (a scheduling choice of this implementation).
 */
int64_t mhc_pre_group_split_tokens(int64_t max_tokens);

/* ------------------------------------------------------------------ backward
 * Gradients are computed in fp32 and rounded once at the store, as the
 * reference's Triton backward kernels do.  Incoming gradients that are NULL
 * count as zero.
 */

/*
 * Post-phase backward, per token:
 *   g_x[j,:] = sum_i h_res[i,j] * g_out[i,:],  g_h_res[i,j] = g_out[i,:] . x[j,:],
 *   g_h_post[i] = g_out[i,:] . f_out,          g_f = sum_i h_post[i] * g_out[i,:].
 * Replaces _PostPhaseFullFn.backward  model/mhc_fused.py:747-772
 *          (its kernel                model/mhc_fused.py:462-526).
 *   g_out, g_x [M, n*C] x_dtype; g_h_res [M, n, n], g_h_post [M, n] h_dtype;
 *   g_f [M, C] f_dtype.  n <= 16.
 */
int mhc_post_bwd(const void* x, int x_dtype, const void* h_res, const void* h_post, int h_dtype,
                 const void* f_out, int f_dtype, const void* g_out, void* g_x, void* g_h_res,
                 void* g_h_post, void* g_f, int64_t M, int n, int C, hipStream_t stream);

/*
 * Post-phase backward without H_res (out = x + h_post (x) f_out): g_x = g_out,
 * so g_x may be NULL (the caller reuses g_out).
 * Replaces _PostPhaseFn.backward  model/mhc_fused_no_hres.py:559-580
 *          (its kernel           model/mhc_fused_no_hres.py:321-360).
 */
int mhc_post_nohres_bwd(const void* h_post, int h_dtype, const void* f_out, int f_dtype,
                        const void* g_out, int x_dtype, void* g_x, void* g_h_post, void* g_f,
                        int64_t M, int n, int C, hipStream_t stream);

/*
 * Pre-phase backward, per token, recomputed from the saved inv_rms and
 * mixes_raw:  g_x (x_dtype) and g_raw [M, FD] fp32, the gradient of each
 * segment's alpha * m + bias (pre and post after the sigmoid derivative,
 * res as given).  g_raw feeds mhc_pre_bwd_weights.
 * mode MHC_MODE_FULL / MHC_MODE_NOHRES: the mHC pre phase; g_sub = d sublayer_in,
 *   g_h_pre, g_h_post, g_h_res_raw as named.
 * mode MHC_MODE_HEAD: MHCHead; g_sub = d out, the other gradients NULL.
 * mode MHC_MODE_RMS: MHCHead with n == 1 (out = x * inv_rms); g_sub = d out,
 *   phi / alphas / biases / mixes_raw / g_raw unused (may be NULL).
 * Replaces _PrePhaseFullFn.backward's kernel  model/mhc_fused.py:271-413, :644-695
 *          _PrePhaseFn.backward's kernel      model/mhc_fused_no_hres.py:150-281, :466-515
 *          _MHCHeadFn.backward's kernel       model/mhc_common.py:200-295, :360-390
 *          the n == 1 RMSNorm head's autograd  model/mhc_common.py:438-442.
 *   bias_post and alpha_res may be NULL where the mode has no such segment;
 *   the four incoming gradients share grad_dtype.
 */
int mhc_pre_bwd(const void* x, int x_dtype, const void* phi, int phi_dtype, const void* alpha_pre,
                const void* bias_pre, const void* alpha_post, const void* bias_post,
                const void* alpha_res, int param_dtype, const float* inv_rms,
                const float* mixes_raw, const void* g_sub, const void* g_h_pre,
                const void* g_h_post, const void* g_h_res_raw, int grad_dtype, void* g_x,
                float* g_raw, int64_t M, int n, int C, int mode, float post_mult, float pre_eps,
                hipStream_t stream);

/* Workspace bytes mhc_pre_bwd_weights needs for (M, n, C, mode). */
int64_t mhc_pre_bwd_weights_workspace_bytes(int64_t M, int n, int C, int mode);

/*
 * Weight gradients of the pre phase from mhc_pre_bwd's g_raw:
 *   g_phi[k, f] = alpha_seg(f) * sum_t x[t, k] * inv_rms[t] * g_raw[t, f]   (phi_dtype)
 *   g_bias_seg  = sum_t g_raw[t, seg]                                       (param_dtype)
 *   g_alpha_seg = sum_t sum_{f in seg} g_raw[t, f] * mixes_raw[t, f]        (param_dtype)
 * Deterministic: token-range partial sums in the workspace, then one
 * reduction.  Any g_alpha_* / g_bias_* may be NULL (skipped).
 * Replaces the grad_W GEMM and alpha / bias reductions of
 *   _PrePhaseFullFn.backward  model/mhc_fused.py:696-711
 *   _PrePhaseFn.backward      model/mhc_fused_no_hres.py:515-525
 *   _MHCHeadFn.backward       model/mhc_common.py:390-398.
 */
int mhc_pre_bwd_weights(const void* x, int x_dtype, const float* inv_rms, const float* mixes_raw,
                        const float* g_raw, const void* alpha_pre, const void* alpha_post,
                        const void* alpha_res, int param_dtype, void* g_phi, int phi_dtype,
                        void* g_alpha_pre, void* g_bias_pre, void* g_alpha_post,
                        void* g_bias_post, void* g_alpha_res, void* g_bias_res, void* workspace,
                        int64_t workspace_bytes, int64_t M, int n, int C, int mode,
                        hipStream_t stream);

/*
 * mhc_pre_bwd_weights without a workspace argument: the token-range partial
 * sums go to a scratch array in device memory that the library holds (32 MiB
 * per device, for the life of the process), so the call allocates nothing.
 * Same arguments and results as mhc_pre_bwd_weights, minus the workspace; the
 * token ranges are capped to what the scratch holds, so sums may group
 * differently (fp32 rounding only).  Rejects shapes whose one-range partials,
 * (n*C*FD + 2*FD) * 4 bytes, exceed the scratch (e.g. n = 16, C = 2048).
 * Calls that overlap on one device share the scratch and race: serialise
 * them (one stream, or events between streams).  Call mhc_init() (or this
 * entry point once, uncaptured) before capturing it in a HIP graph.
 * No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).
 */
int mhc_pre_bwd_weights_noalloc(const void* x, int x_dtype, const float* inv_rms,
                                const float* mixes_raw, const float* g_raw, const void* alpha_pre,
                                const void* alpha_post, const void* alpha_res, int param_dtype,
                                void* g_phi, int phi_dtype, void* g_alpha_pre, void* g_bias_pre,
                                void* g_alpha_post, void* g_bias_post, void* g_alpha_res,
                                void* g_bias_res, int64_t M, int n, int C, int mode,
                                hipStream_t stream);

/*
 * Largest Sinkhorn iteration count mhc_sinkhorn_bwd accepts for n (64 for
 * n in {2, 4, 8}, 30 otherwise; 0 for n outside [1, 16]).  The forward
 * kernels take any count; a caller that will need gradients checks this
 * before the forward.  No reference counterpart: the reference's backward
 * recomputes the forward under autograd (model/mhc_fused.py:131-137) and has
 * no limit.
 */
int mhc_sinkhorn_bwd_max_iters(int n);

/*
 * Sinkhorn-Knopp backward: g_in = d output / d input of mhc_sinkhorn_fwd's
 * schedule, by recomputing the forward iterates (fp32).  n <= 16;
 * iters <= 64 for n in {2, 4, 8}, <= 30 otherwise (the iterates live in LDS).
 * Replaces _SinkhornFn.backward  model/mhc_fused.py:131-137.
 */
int mhc_sinkhorn_bwd(const void* m_in, int in_dtype, const void* g_out, int g_dtype, void* g_in,
                     int gi_dtype, int64_t batch, int n, int iters, float eps, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_AMD_H_ */
