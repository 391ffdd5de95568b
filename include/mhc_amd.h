/*
 * mhc_amd.h -- C ABI of the MI355X (gfx950) mHC forward kernels.
 *
 * Every entry point takes raw device pointers, plain sizes and a hipStream_t,
 * enqueues its kernels on that stream and returns without synchronising.
 * The caller allocates every output (as the reference's autograd Functions do
 * with torch.empty); the library never allocates or frees device memory and
 * keeps no state between calls, so calls are re-entrant and capturable.
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

/* ABI revision (bumped on any signature change). */
int mhc_abi_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* mhc_last_error(void);

/*
 * Size in bytes of the MFMA operand image of phi for (n, C, mode), or 0 when
 * that shape has no MFMA kernel (n not in {1,2,4,8}, C % 8 != 0, C > 1024,
 * or MHCHead with n == 1).  Host-only, no device work.
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
 *   phi_packed   mhc_phi_pack image of phi, or NULL (then a VALU kernel runs)
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
 */
int mhc_pre_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype, const void* phi_packed,
                const void* alpha_pre, const void* bias_pre, const void* alpha_post,
                const void* bias_post, const void* alpha_res, const void* bias_res,
                int param_dtype, void* sublayer_in, void* h_pre, void* h_post, void* h_res_raw,
                void* h_res, float* inv_rms, float* mixes_raw, int64_t M, int n, int C,
                float post_mult, float pre_eps, float rms_eps, int sinkhorn_iters,
                float sinkhorn_eps, hipStream_t stream);

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
                       float rms_eps, hipStream_t stream);

/*
 * Post phase: out[t,i,:] = sum_j h_res[t,i,j] * x[t,j,:] + h_post[t,i] * f_out[t,:].
 * Replaces _PostPhaseFullFn.forward  model/mhc_fused.py:720-744
 *          (its kernel               model/mhc_fused.py:416-459).
 *   x [M, n*C] x_dtype; h_res [M, n, n] and h_post [M, n] h_dtype;
 *   f_out [M, C] f_dtype; out [M, n*C] x_dtype (must not alias x).
 */
int mhc_post_fwd(const void* x, int x_dtype, const void* h_res, const void* h_post, int h_dtype,
                 const void* f_out, int f_dtype, void* out, int64_t M, int n, int C,
                 hipStream_t stream);

/*
 * Post phase without H_res: out = x + h_post (x) f_out.
 * Replaces _PostPhaseFn.forward  model/mhc_fused_no_hres.py:535-556
 *          (its kernel           model/mhc_fused_no_hres.py:284-316).
 */
int mhc_post_nohres_fwd(const void* x, int x_dtype, const void* h_post, int h_dtype,
                        const void* f_out, int f_dtype, void* out, int64_t M, int n, int C,
                        hipStream_t stream);

/*
 * MHCHead exit: out = sum_i (sigmoid(alpha * (x_norm @ phi)_i + bias_i) + pre_eps) * x_i,
 * phi [n*C, n], alpha shape (1,), bias [n].  For n == 1 it is the plain
 * RMSNorm out = x * inv_rms (phi, alpha, bias ignored and may be NULL).
 * Replaces _MHCHeadFn.forward     model/mhc_common.py:315-357
 *          (its kernel            model/mhc_common.py:128-195)
 *          and MHCHead.forward's n == 1 branch  model/mhc_common.py:438-442.
 *   out [M, C] x_dtype; inv_rms [M], mix_raw [M, n] fp32 optional.
 */
int mhc_head_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                 const void* phi_packed, const void* alpha, const void* bias, int param_dtype,
                 void* out, float* inv_rms, float* mix_raw, int64_t M, int n, int C, float pre_eps,
                 float rms_eps, hipStream_t stream);

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

#ifdef __cplusplus
}
#endif

#endif /* MHC_AMD_H_ */
