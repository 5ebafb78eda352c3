/*
 * velograd_kernels.h — C ABI of the MI355X (gfx950) fused RMSNorm + residual-add kernels.
 *
 * These entry points sit below the Python functions `fused_rmsnorm_residual_forward`,
 * `fused_rmsnorm_residual_backward` and `fused_rmsnorm_residual` of `velograd_amd.kernels`,
 * which keep the call signatures of the reference's `velograd.kernels`
 * (python/velograd/kernels/fused.py:28-66, python/velograd/kernels/__init__.py:19-32).
 *
 * Conventions (follow the reference's only C ABI, include/velograd/aot_compiler.h:74-90):
 *   - `velograd_` prefix, default symbol visibility, `int32_t` status return.
 *   - 0 = success; negative = argument error (nothing was launched); positive = the hipError_t
 *     reported by the HIP runtime right after the launch.  The text of the last error of the
 *     calling thread is returned by velograd_kernels_last_error().
 *   - The library never allocates or frees device memory and never synchronises the host:
 *     every buffer (outputs and the backward workspace) belongs to the caller, and every
 *     launch is asynchronous on `hip_stream` (a hipStream_t; NULL = the null stream).  The one
 *     device array the library holds is the fixed 16 MiB scratch of
 *     velograd_rmsnorm_residual_bwd_noalloc, placed with its code on each GPU it runs on.
 *   - Tensors are row-major [rows, dim] with unit stride along dim; `ld_*` is the row stride in
 *     elements.  Rows are independent; the normalisation runs over dim.
 *   - Results are deterministic: the same inputs on the same device give bitwise identical
 *     outputs, dweight included (no floating-point atomics anywhere).
 *   - Output buffers must not overlap input buffers.
 */
#ifndef VELOGRAD_KERNELS_H
#define VELOGRAD_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VELOGRAD_API __attribute__((visibility("default")))

/* Element types of activations (`dtype`) and of the weight vector (`w_dtype`). */
#define VELOGRAD_DTYPE_F32 0
#define VELOGRAD_DTYPE_F16 1
#define VELOGRAD_DTYPE_BF16 2

/* Negative status codes (argument errors, nothing launched). */
#define VELOGRAD_ERR_INVALID_ARGUMENT (-1)
#define VELOGRAD_ERR_UNSUPPORTED_DTYPE (-2)
#define VELOGRAD_ERR_WORKSPACE_TOO_SMALL (-3)
#define VELOGRAD_ERR_DEVICE_QUERY (-4)

/*
 * Forward: h = x + residual; inv_rms = 1 / sqrt(mean(h^2) + eps); y = (h * inv_rms) * weight.
 * Replaces fused_rmsnorm_residual_forward (python/velograd/kernels/fused.py:28-46).
 *
 *   x, residual : [rows, dim] in `dtype`; residual may be NULL (then h is x, as fused.py:39).
 *   weight      : [dim] in `w_dtype` (= dtype or F32); NULL means no scale (fused.py:44-45).
 *   y           : [rows, dim] in `dtype` (required).
 *   h           : [rows, dim] in `dtype`; may be NULL (not written).  Ignored when residual is
 *                 NULL, since h is x itself then.
 *   inv_rms     : [rows] fp32; may be NULL (not written).
 *   eps         : added in fp32 to mean(h^2), as NumPy adds a Python float to a float32 array.
 * All arithmetic is fp32; stores round to nearest even.  h feeds the row statistic and y
 * unrounded (fp32), as the reference computes both from the fp32 sum.
 */
VELOGRAD_API int32_t velograd_rmsnorm_residual_fwd(
    const void* x, const void* residual, const void* weight,
    void* y, void* h, float* inv_rms,
    int64_t rows, int64_t dim,
    int64_t ld_x, int64_t ld_res, int64_t ld_y, int64_t ld_h,
    int32_t dtype, int32_t w_dtype, float eps, void* hip_stream);

/*
 * RMSNorm with a floor on the mean square, as the reference's module computes it
 * (`velograd.nn.RMSNorm.forward`, python/velograd/nn.py:338-355), optionally after the residual
 * add its model performs first (`h = x + attn_out; ffn_norm(h)`, models/llama.py:52-54):
 *   h = x + residual (residual may be NULL: h is x);  mean_sq = max(min_mean_sq, mean(h^2));
 *   inv_rms = 1 / sqrt(mean_sq + eps);  y = (h * inv_rms) * w
 * The reference floors at 1e-12 (nn.py:349).  As in Python's max, a NaN mean square becomes the
 * floor (the NaN elements of y stay NaN, the others stay finite).  min_mean_sq must be finite and
 * >= 0; 0 gives velograd_rmsnorm_residual_fwd exactly.  The module's backward (nn.py:357-383) is
 * velograd_rmsnorm_residual_bwd with saved = h, saved_is_h = 1.
 * Arguments as velograd_rmsnorm_residual_fwd.
 */
VELOGRAD_API int32_t velograd_rmsnorm_fwd(
    const void* x, const void* residual, const void* weight,
    void* y, void* h, float* inv_rms,
    int64_t rows, int64_t dim,
    int64_t ld_x, int64_t ld_res, int64_t ld_y, int64_t ld_h,
    int32_t dtype, int32_t w_dtype, float eps, float min_mean_sq, void* hip_stream);

/*
 * The reference model's attention-branch input in one pass: its module RMSNorm followed by its
 * interleaved RoPE of the whole hidden vector (`normed_attn = attention_norm(x);
 * F.apply_rotary_emb(normed_attn)`, python/velograd/models/llama.py:48-49, with nn.py:338-355
 * and functional.py:287-315), optionally after a residual add:
 *   h = x + residual;  mean_sq = max(min_mean_sq, mean(h^2));  n = h / sqrt(mean_sq + eps) * w
 *   y_2i, y_2i+1 = n_2i cos - n_2i+1 sin, n_2i sin + n_2i+1 cos at angle pos * base^(-2i/dim)
 * where pos = row % seq (rows hold [outer, seq] positions in order).  y is rotated in fp32
 * before its single rounding.  inv_rms is the statistic of the norm, so the backward is
 * velograd_rope(pairing = VELOGRAD_ROPE_INTERLEAVED, inverse = 1) of grad_y followed by
 * velograd_rmsnorm_residual_bwd with saved = h, or both in one pass:
 * velograd_rmsnorm_rope_bwd.  No counterpart in the reference, which makes two passes (and two
 * Python loops); it replaces that pair.
 *
 *   dim  : even.   seq : >= 1 and dividing rows.   base : finite, > 0.
 * Other arguments as velograd_rmsnorm_fwd.
 */
VELOGRAD_API int32_t velograd_rmsnorm_rope_fwd(
    const void* x, const void* residual, const void* weight,
    void* y, void* h, float* inv_rms,
    int64_t rows, int64_t dim,
    int64_t ld_x, int64_t ld_res, int64_t ld_y, int64_t ld_h,
    int64_t seq, int32_t dtype, int32_t w_dtype, float eps, float min_mean_sq, float base,
    void* hip_stream);

/*
 * Forward with an fp8 output epilogue: h and inv_rms as velograd_rmsnorm_residual_fwd, while y
 * leaves as fp8 E4M3 codes with one dequantisation scale per row, ready for an fp8 GEMM:
 *   amax = max |y| over the row (fp32 y, before any rounding; NaN if the row holds a NaN)
 *   y_scale[row] = amax / 448                     (fp32; 448 is E4M3's largest finite value)
 *   y_fp8 = e4m3(y * inv), inv = 1 / y_scale in fp32, or inv = 1 where y_scale is below the
 *           smallest normal float (an all-zero row)
 * e4m3 rounds to nearest even and saturates to +-448; NaN maps to the NaN code with its sign.
 * The format is OCP "e4m3fn" (bias 7, no infinities, S.1111.111 = NaN), the E4M3 that the
 * reference enumerates and decodes (include/velograd/kernels.h:29-37 PrecisionMode::FP8_E4M3,
 * :58-73 fp8_e4m3_to_f32).  The reference has no fused quantising forward; this replaces the
 * pair "fused_rmsnorm_residual_forward (fused.py:28-46) then a separate quantisation pass".
 * Dequantise as y ~= float(y_fp8) * y_scale.
 *
 *   y_fp8   : [rows, dim] bytes; ld_y is its row stride in bytes.
 *   y_scale : [rows] fp32 (required).
 * Other arguments as velograd_rmsnorm_residual_fwd.
 */
VELOGRAD_API int32_t velograd_rmsnorm_residual_fwd_fp8(
    const void* x, const void* residual, const void* weight,
    uint8_t* y_fp8, float* y_scale, void* h, float* inv_rms,
    int64_t rows, int64_t dim,
    int64_t ld_x, int64_t ld_res, int64_t ld_y, int64_t ld_h,
    int32_t dtype, int32_t w_dtype, float eps, void* hip_stream);

/* Element formats of the MX (OCP Microscaling) forward. */
#define VELOGRAD_MX_E4M3 0 /* MXFP8: fp8 E4M3 elements */
#define VELOGRAD_MX_E2M1 1 /* MXFP4: fp4 E2M1 elements, two per byte */

/*
 * Forward with an MX output epilogue, the block-scaled layout of gfx950's scaled MFMA: h and
 * inv_rms as velograd_rmsnorm_residual_fwd, while y leaves in blocks of 32 consecutive elements
 * of a row that share one E8M0 scale 2^s:
 *   amax = max |y| over the block (fp32 y, before any rounding)
 *   s    = floor(log2(amax)) - emax, emax = 8 (E4M3) or 2 (E2M1), clamped to [-127, 127];
 *          scale code s + 127; code 0 for an all-zero block; 0xFF (NaN) and zero element codes
 *          for a block whose amax is not finite
 *   element codes = round-to-nearest-even, saturating (+-448 / +-6) codes of y * 2^-s
 * (OCP Microscaling Formats v1.0).  E2M1 nibbles are packed two per byte, the even element in
 * the low nibble, and the scales are one byte per block: the layout the reference decodes with
 * its E2M1 table (include/velograd/kernels.h:47-51, 97-101, 339-347).  No counterpart in the
 * reference's NumPy path; it replaces "fused_rmsnorm_residual_forward (fused.py:28-46), then a
 * separate MX quantisation pass".
 *
 *   dim       : a multiple of 32.
 *   y_q       : [rows, dim] bytes (E4M3) or [rows, dim / 2] bytes (E2M1); ld_yq in bytes.
 *   y_scales  : [rows, dim / 32] E8M0 bytes; ld_scales in bytes.
 *   mx_format : VELOGRAD_MX_E4M3 or VELOGRAD_MX_E2M1.
 * Other arguments as velograd_rmsnorm_residual_fwd.
 */
VELOGRAD_API int32_t velograd_rmsnorm_residual_fwd_mx(
    const void* x, const void* residual, const void* weight,
    uint8_t* y_q, uint8_t* y_scales, void* h, float* inv_rms,
    int64_t rows, int64_t dim,
    int64_t ld_x, int64_t ld_res, int64_t ld_yq, int64_t ld_scales, int64_t ld_h,
    int32_t dtype, int32_t w_dtype, int32_t mx_format, float eps, void* hip_stream);

/*
 * Backward of the forward above.
 * Replaces fused_rmsnorm_residual_backward (python/velograd/kernels/fused.py:48-66):
 *   gw = grad_y * weight; m = mean(gw * xhat); dx = inv_rms * (gw - xhat * m);
 *   dweight = sum over rows of grad_y * xhat.
 *
 *   grad_y      : [rows, dim] in `dtype`.
 *   saved       : [rows, dim] in `dtype`: xhat = h * inv_rms (the reference's `normed_input`)
 *                 when saved_is_h == 0, or h itself when saved_is_h != 0 (then xhat = h * inv_rms
 *                 is formed in fp32 in registers; same bytes moved).
 *   weight      : [dim] in `w_dtype`, or NULL (gw = grad_y; dweight is then not computed).
 *   inv_rms     : [rows] fp32, as written by the forward.
 *   grad_h      : optional [rows, dim] in `dtype`: gradient that reaches h from its other
 *                 consumer (in a pre-norm block, the next residual add, models/llama.py:48-56);
 *                 when given, dx = backward + grad_h, added in fp32 before the one rounding.
 *                 No counterpart in the reference's backward (fused.py:48-66), which stops at
 *                 the norm.  dx may be grad_h itself (accumulate in place, same row stride).
 *   dx          : [rows, dim] in `dtype` (required).  Since h = x + residual, it is also the
 *                 gradient of residual.
 *   dres        : optional [rows, dim] second copy of dx for callers that need two buffers.
 *   dweight     : [dim] fp32, or NULL.  Reduced in two deterministic stages through `workspace`.
 *   workspace   : device scratch of at least
 *                 velograd_rmsnorm_residual_bwd_workspace_bytes(rows, dim, device) bytes,
 *                 16-byte aligned; may be NULL when dweight is NULL.
 */
VELOGRAD_API int32_t velograd_rmsnorm_residual_bwd(
    const void* grad_y, const void* saved, int32_t saved_is_h,
    const void* weight, const float* inv_rms, const void* grad_h,
    void* dx, void* dres, float* dweight,
    void* workspace, size_t ws_bytes,
    int64_t rows, int64_t dim,
    int64_t ld_g, int64_t ld_saved, int64_t ld_grad_h, int64_t ld_dx, int64_t ld_dres,
    int32_t dtype, int32_t w_dtype, void* hip_stream);

/*
 * velograd_rmsnorm_residual_bwd without a workspace argument: the allocation-free variant.
 * No counterpart in the reference.  It is for callers that cannot allocate device memory or
 * size a workspace: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  It allocates nothing and calls no allocating routine; the dweight partial rows
 * go to a scratch array of 16 MiB that the library holds on each GPU it runs on until the
 * process ends.
 *
 *   Arguments and results as velograd_rmsnorm_residual_bwd (same kernels, so bitwise the same
 *   outputs), minus `workspace` and `ws_bytes`.
 *   Limit: returns VELOGRAD_ERR_WORKSPACE_TOO_SMALL, launching nothing, when dweight would
 *   need more than the 16 MiB, i.e. one fp32 row of dim per partial.  With the default launch
 *   plans on a 256-CU MI355X that is 256 partials for 16-byte-aligned rows up to dim 16384
 *   bf16/fp16 or 8192 fp32, for bf16/fp16 rows of 8n + 4 elements on 8-byte boundaries up
 *   to dim 4100, and for other rows up to dim 4096 (the element-strided kernel); wider rows of
 *   those kinds take the generic path with min(rows, 4 per CU) partials, refused when those
 *   pass 16 MiB (at 1024 or more rows, any dim above 4096).  The VELOGRAD_BWD_* tuning
 *   variables change the plans, and with them which shapes are refused.
 *   Calls that overlap on one GPU (several streams or host threads at once) share the scratch
 *   and race: serialise them.  The scratch keeps the last call's contents; nothing in it has
 *   to start at zero.
 */
VELOGRAD_API int32_t velograd_rmsnorm_residual_bwd_noalloc(
    const void* grad_y, const void* saved, int32_t saved_is_h,
    const void* weight, const float* inv_rms, const void* grad_h,
    void* dx, void* dres, float* dweight,
    int64_t rows, int64_t dim,
    int64_t ld_g, int64_t ld_saved, int64_t ld_grad_h, int64_t ld_dx, int64_t ld_dres,
    int32_t dtype, int32_t w_dtype, void* hip_stream);

/*
 * Backward of velograd_rmsnorm_rope_fwd in one pass: grad_y (the gradient of the rotated y) is
 * rotated back pair by pair in registers, (g_2i, g_2i+1) -> (g_2i cos + g_2i+1 sin,
 * g_2i+1 cos - g_2i sin) at the forward's angles (the rotation's backward, functional.py:316-345),
 * then the norm's backward runs on it as velograd_rmsnorm_residual_bwd does with saved = h
 * (nn.py:357-383 for the module form; fused.py:48-66):
 *   dx = inv_rms * (gw - xhat * mean(gw * xhat)),  gw = g * w,  xhat = h * inv_rms,
 *   dweight = sum over rows of g * xhat.
 * One HBM pass over grad_y, h and dx instead of two over grad_y.  With a residual in the
 * forward, dx is also the gradient of the residual.  No counterpart in the reference (two
 * passes there).
 *
 *   grad_y, h, dx : [rows, dim] in `dtype` (unit stride along dim; row strides ld_*).
 *   weight, inv_rms, dweight, workspace, ws_bytes : as velograd_rmsnorm_residual_bwd (the size
 *                 query covers this entry point's plans too).
 *   seq, base     : as velograd_rmsnorm_rope_fwd (even dim, seq >= 1 dividing rows, finite
 *                 base > 0).
 */
VELOGRAD_API int32_t velograd_rmsnorm_rope_bwd(
    const void* grad_y, const void* h, const void* weight, const float* inv_rms,
    void* dx, float* dweight, void* workspace, size_t ws_bytes,
    int64_t rows, int64_t dim, int64_t ld_g, int64_t ld_h, int64_t ld_dx,
    int64_t seq, int32_t dtype, int32_t w_dtype, float base, void* hip_stream);

/*
 * Workspace needed by velograd_rmsnorm_residual_bwd and velograd_rmsnorm_rope_bwd for dweight
 * on `device` (a HIP device ordinal).  No counterpart in the reference, whose NumPy backward allocates its own
 * temporaries (fused.py:58-65); returns 0 if the device cannot be queried.
 */
VELOGRAD_API size_t velograd_rmsnorm_residual_bwd_workspace_bytes(int64_t rows, int64_t dim,
                                                                  int32_t device);

/* Pairings of a head vector's elements for velograd_rope. */
#define VELOGRAD_ROPE_HALF 0        /* (j, j + rot_dim/2): fused.py, fused_kernels.cu */
#define VELOGRAD_ROPE_INTERLEAVED 1 /* (2j, 2j + 1): functional.apply_rotary_emb, ops.rs */

/*
 * Rotary position embedding on one tensor (call once for q and once for k), laid out as
 * [outer, seq, heads, dim]; the position of x[o, s, h, :] is s.  For j < rot_dim / 2,
 *   freq_j = 1 / theta^(2j / rot_dim), angle = s * freq_j (fp32 for VELOGRAD_ROPE_HALF as
 *   fused.py:98-103 forms it; double, reduced exactly before a float32 sincospi, for
 *   VELOGRAD_ROPE_INTERLEAVED as functional.py:302-305 does), and the pair (a, b) of j
 *   becomes (a cos - b sin, a sin + b cos); elements rot_dim .. dim-1 are copied.
 * pairing VELOGRAD_ROPE_HALF: (a, b) = (x_j, x_{j + rot_dim/2}).  Replaces fused_rope_forward
 *   (python/velograd/kernels/fused.py:72-130; positions fused.py:96-98, angles :98-103, copied
 *   tail :119-120) and the reference's CUDA kernel (src/cuda/fused_kernels.cu:145-181).
 * pairing VELOGRAD_ROPE_INTERLEAVED: (a, b) = (x_{2j}, x_{2j+1}).  Replaces
 *   apply_rotary_emb (python/velograd/functional.py:287-315, the RoPE the reference's LLaMA
 *   model applies, models/llama.py:49; there x is [..., seq, dim]: heads = 1, rot_dim = dim)
 *   and rotary_pos_embedding_forward (src/ops.rs:465-499).
 *
 *   x, out   : [outer, seq, heads, dim] contiguous in `dtype`; out may be x itself (in place)
 *              but must not otherwise overlap it.
 *   rot_dim  : the rotated width (the reference's head_dim): even, 2 <= rot_dim <= dim;
 *              rot_dim <= 8192 unless the pairing is interleaved on 16-byte aligned rows of a
 *              16-byte multiple (any rot_dim there).
 *   theta    : the frequency base (> 0).
 *   inverse  : nonzero rotates by -angle: the backward (grad_x from grad_out), the rotary
 *              backward of src/ops.rs:501-530 and functional.py:316-345.
 *   pairing  : VELOGRAD_ROPE_HALF or VELOGRAD_ROPE_INTERLEAVED.
 */
VELOGRAD_API int32_t velograd_rope(
    const void* x, void* out,
    int64_t outer, int64_t seq, int64_t heads, int64_t dim,
    int64_t rot_dim, float theta, int32_t inverse, int32_t pairing,
    int32_t dtype, void* hip_stream);

/* Text of the calling thread's last error ("" if none).  No counterpart in the reference. */
VELOGRAD_API const char* velograd_kernels_last_error(void);

/* Library version string; mirrors velograd_get_version (include/velograd/aot_compiler.h:89). */
VELOGRAD_API const char* velograd_kernels_version(void);

#ifdef __cplusplus
}
#endif

#endif /* VELOGRAD_KERNELS_H */
