/*
 * joyomni_hip.h — C ABI of the MI355X (gfx950) joyomni_ops kernel library.
 *
 * libjoyomni_hip.so exports these entry points. Every argument is a plain
 * pointer, an integer or a float; no torch or HIP type appears, so the header
 * can be bound from ctypes, cgo, JNI or N-API as easily as from C++.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers on the device that owns
 *     `stream`; that device must be current on the calling thread.
 *   - `stream` is a hipStream_t passed as void*; NULL selects the null stream.
 *     Work is enqueued asynchronously on it. No entry point synchronizes,
 *     allocates device memory or queries device properties after its first
 *     call on a device, so all of them are safe inside HIP graph capture.
 *   - Strides are in ELEMENTS of the tensor they describe. The innermost
 *     dimension is always contiguous. A row stride of 0 broadcasts one row.
 *   - Element types are selected with JO_DTYPE_*; fp8 outputs are OCP
 *     float8 e4m3fn bytes (the format of torch.float8_e4m3fn).
 *   - The return value is a status: JO_OK (0) or a JO_ERR_* code. On error
 *     nothing is enqueued (validation errors) or the launch failed
 *     (JO_ERR_HIP); jo_last_error() returns a message for the calling thread.
 *
 * Which reference function each entry point replaces is given in its comment
 * as path:line into jd-opensource/JoyAI-Video-Edit.
 */
#ifndef JOYOMNI_HIP_H
#define JOYOMNI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JO_ABI_VERSION 4

/* Status codes. */
#define JO_OK 0
#define JO_ERR_INVALID 1     /* bad pointer, shape, stride, alignment or enum   */
#define JO_ERR_UNSUPPORTED 2 /* valid request this build has no kernel for      */
#define JO_ERR_HIP 3         /* the HIP runtime reported an error at launch     */

/* Element types of bf16/fp16/fp32 tensors. */
#define JO_DTYPE_F32 0
#define JO_DTYPE_F16 1
#define JO_DTYPE_BF16 2

/* norm_type values; the integers are the reference's own
 * (deploy/joyomni_ops/csrc/fused_norm_scale_shift.cu:25,
 *  deploy/joyomni_ops/joyomni_ops/__init__.py:38-41). */
#define JO_NORM_LAYER 0
#define JO_NORM_RMS 1

/* Message describing the last error on the calling thread ("" if none). */
const char* jo_last_error(void);

/* JO_ABI_VERSION of the loaded library. */
int jo_abi_version(void);

/* Launch-shape knobs. Each selects how a kernel is spread over waves, never
 * what it computes: results are identical under every setting. The value is
 * -1 (the library's own choice) unless the environment variable named below
 * was set when the library was loaded, or jo_set_launch_override() changed it.
 *   JO_KNOB_QK_SPLIT    waves per token of the QK norm + RoPE kernels: 1, 2,
 *                       4, 6 or 8 (env JO_QK_SPLIT)
 *   JO_KNOB_KV_SPLIT    1 = K and V of a KV-pool row on one wave, 2 = on two
 *                       (env JO_KV_SPLIT)
 *   JO_KNOB_GEMM_SHAPE  FP8 GEMM tile: 0 = 256x256, 1 = 256x128, 2 = the
 *                       register-staged kernel, 3 = 224x256, 4 = 224x128,
 *                       5 = 128x128 and 6 = 64x64 (four waves), 7 = 128x256
 *                       (eight waves), 8 = 64x128, 9 = 128x192 and 10 =
 *                       128x96 (four waves), 11 = 64x96 (two waves; 5-11
 *                       need K % 128 == 0, else the
 *                       register-staged kernel runs) (env JO_GEMM_SHAPE)
 *   JO_KNOB_GEMM_SPLIT  FP8 GEMM K split: 1 (none), 2, 4 or 8 workgroups per
 *                       tile, taken by the 128x128 and 64x64 tiles when
 *                       jo_fp8_scaled_mm_ws has the workspace for it and
 *                       K % (128 x split) == 0 (env JO_GEMM_SPLIT)
 * No reference counterpart (tuning and test hook). */
#define JO_KNOB_QK_SPLIT 0
#define JO_KNOB_KV_SPLIT 1
#define JO_KNOB_GEMM_SHAPE 2
#define JO_KNOB_GEMM_SPLIT 3

/* Sets knob `knob` to `value` (-1 restores the automatic choice) for every
 * later launch in the process. Returns JO_ERR_INVALID for an unknown knob or
 * a value the knob does not list above (an environment value the knob does
 * not accept is ignored at load, with a message on stderr). */
int jo_set_launch_override(int knob, int value);

/* ------------------------------------------------------------------------
 * Per-token FP8 e4m3 quantization.
 * Replaces joyomni_ops::sgl_per_token_quant_fp8
 *   (deploy/joyomni_ops/csrc/per_token_quant_fp8.cu:148-176; kernel :43-83).
 * For each row r:  s[r] = max_j |x[r,j]| / 448  (IEEE fp32 division),
 *   inv = (s[r] == 0) ? 0 : 1 / s[r],
 *   q[r,j] = e4m3fn_rne(min(max(x[r,j] * inv, -448), 448)).
 * NaN inputs are ignored by the max and quantize to +448, as in the reference.
 * input: [num_tokens, hidden_dim] bf16 or fp16 (dtype), row stride in_stride.
 * output_q: fp8 bytes, row stride q_stride. output_s: fp32 [num_tokens].
 * hidden_dim % 4 == 0 (the reference's requirement).
 * ------------------------------------------------------------------------ */
int jo_sgl_per_token_quant_fp8(const void* input, int dtype, int64_t num_tokens,
                               int64_t hidden_dim, int64_t in_stride, void* output_q,
                               int64_t q_stride, float* output_s, void* stream);

/* ------------------------------------------------------------------------
 * Fused per-head QK RMSNorm + interleaved-pair RoPE from bf16 cos/sin tables,
 * in place on q and k.
 * Replaces joyomni_ops::fused_qk_norm_rope_3d_paired
 *   (deploy/joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:179-208;
 *    kernel :56-143, launch :145-175).
 * For every head vector x (head_dim elements) of q (weight q_weight) and of
 * k (weight k_weight) at sequence position n:
 *   r = 1/sqrt(sum(x^2)/head_dim + eps);  e_d = x_d * (r * w_d)
 *   (e_2i, e_2i+1) <- (e_2i c - e_2i+1 s, e_2i s + e_2i+1 c),
 *   c = cos[n, i], s = sin[n, i]; one bf16 rounding at the end.
 * q, k: bf16 [batch, seq_len, num_heads, head_dim] with the given batch and
 * token strides; heads of a token are contiguous (head stride head_dim).
 * q_weight, k_weight: bf16 [head_dim]. cos, sin: bf16 [seq_len, head_dim/2]
 * contiguous. head_dim in {64, 128, 256}.
 * ------------------------------------------------------------------------ */
int jo_fused_qk_norm_rope_3d_paired(void* q, void* k, int64_t batch, int64_t seq_len,
                                    int64_t num_heads, int64_t head_dim,
                                    int64_t q_batch_stride, int64_t q_token_stride,
                                    int64_t k_batch_stride, int64_t k_token_stride, float eps,
                                    const void* q_weight, const void* k_weight,
                                    const void* cos, const void* sin, void* stream);

/* ------------------------------------------------------------------------
 * Same normalization and rotation as jo_fused_qk_norm_rope_3d_paired, with
 * the rotation angles computed in registers from the token's 3D grid
 * position instead of read from [seq_len, head_dim/2] tables.
 * No reference counterpart with this signature: it computes what the
 * reference's table builders feed the paired kernel
 *   (deploy/xvideo/models/dit/rope.py:31-52, dit.py:745-783 for the 3D
 *    angles, dit.py:785-809,918-933 for the source-id rotation).
 * Token n of the sequence sits in frame f = n / (grid_h*grid_w) at
 *   t = t0 + f,  h = (n % (grid_h*grid_w)) / grid_w,  w = n % grid_w.
 * Pair i (0 <= i < head_dim/2) uses axis t for i < pairs_t, h for
 * i < pairs_t + pairs_h, w otherwise; its angle is pos_axis * freqs[i]
 * (fp32 product). If source_id != 0 the pair is further rotated by
 * source_id * freqs[head_dim/2 + i] by angle addition.
 * freqs: HOST fp32 [2, head_dim/2] (axis frequencies, source-id
 * frequencies), copied into the launch's kernel arguments: nothing is
 * copied to the device, so a call needs no setup and can be captured into
 * a HIP graph on first use. The second row is used only when source_id != 0.
 * ------------------------------------------------------------------------ */
int jo_fused_qk_norm_rope_3d_grid(void* q, void* k, int64_t batch, int64_t seq_len,
                                  int64_t num_heads, int64_t head_dim,
                                  int64_t q_batch_stride, int64_t q_token_stride,
                                  int64_t k_batch_stride, int64_t k_token_stride, float eps,
                                  const void* q_weight, const void* k_weight,
                                  const float* freqs, int32_t pairs_t, int32_t pairs_h,
                                  int32_t grid_h, int32_t grid_w, int32_t t0,
                                  float source_id, void* stream);

/* ------------------------------------------------------------------------
 * jo_fused_qk_norm_rope_3d_paired / _grid with a second output: the
 * pre-RoPE normalized K, written to k_stage in the same pass that rotates q
 * and k in place, so K is read once:
 *   k_stage[b, n, h, :] = bf16((x * r') * k_weight),
 *   r' = 1 / sqrt(sum(x^2) / head_dim + eps)   (separate IEEE operations)
 * for every head vector x of k — bit for bit the row that rmsnorm_qk_bf16
 * (jo_rmsnorm_heads with round_first = 0, or jo_rmsnorm on the rows)
 * returns for the same k.
 * Replaces the pair of calls of the DiT's pre-RoPE KV-cache path
 *   (deploy/xvideo/models/dit/dit.py:360-370: rmsnorm_qk_bf16 of the K slice,
 *    then fused_qk_norm_rope_3d; sgl_fused_ops.py:57-111), whose first call
 *    re-reads K. The stage rows feed the graph runner's pre-RoPE K buffers
 *    (deploy/xvideo/serving/graph_runner.py:56-59,93-95).
 * k_stage: bf16 [batch, seq_len, num_heads, head_dim] with the given batch and
 * token strides (heads contiguous), 16-byte aligned, not overlapping q or k.
 * The other arguments are those of the entry point without _kstage.
 * ------------------------------------------------------------------------ */
int jo_fused_qk_norm_rope_3d_paired_kstage(void* q, void* k, void* k_stage, int64_t batch,
                                           int64_t seq_len, int64_t num_heads, int64_t head_dim,
                                           int64_t q_batch_stride, int64_t q_token_stride,
                                           int64_t k_batch_stride, int64_t k_token_stride,
                                           int64_t stage_batch_stride,
                                           int64_t stage_token_stride, float eps,
                                           const void* q_weight, const void* k_weight,
                                           const void* cos, const void* sin, void* stream);
int jo_fused_qk_norm_rope_3d_grid_kstage(void* q, void* k, void* k_stage, int64_t batch,
                                         int64_t seq_len, int64_t num_heads, int64_t head_dim,
                                         int64_t q_batch_stride, int64_t q_token_stride,
                                         int64_t k_batch_stride, int64_t k_token_stride,
                                         int64_t stage_batch_stride, int64_t stage_token_stride,
                                         float eps, const void* q_weight, const void* k_weight,
                                         const float* freqs, int32_t pairs_t, int32_t pairs_h,
                                         int32_t grid_h, int32_t grid_w, int32_t t0,
                                         float source_id, void* stream);

/* ------------------------------------------------------------------------
 * Grid-mode QK norm + RoPE that writes the rotated K straight into a frame
 * ring buffer: q is updated in place, k is only read, and the rotated head
 * vectors of k for frame f go to cache frame slot (slot_start + f) % cache_slots,
 * i.e. cache token ((slot_start + f) % cache_slots) * grid_h*grid_w + (n % (grid_h*grid_w)).
 * No reference counterpart: it fuses the reference's pre-RoPE K staging and
 * RoPE-at-commit pool write
 *   (deploy/xvideo/serving/graph_runner.py:49-60,137-142; dit.py:360-363).
 * k_cache: bf16 [batch, cache_slots*grid_h*grid_w, num_heads, head_dim] with
 * the given batch and token strides.
 * ------------------------------------------------------------------------ */
int jo_fused_qk_norm_rope_3d_kvcache(void* q, const void* k, void* k_cache, int64_t batch,
                                     int64_t seq_len, int64_t num_heads, int64_t head_dim,
                                     int64_t q_batch_stride, int64_t q_token_stride,
                                     int64_t k_batch_stride, int64_t k_token_stride,
                                     int64_t cache_batch_stride, int64_t cache_token_stride,
                                     int64_t cache_slots, int64_t slot_start, float eps,
                                     const void* q_weight, const void* k_weight,
                                     const float* freqs, int32_t pairs_t, int32_t pairs_h,
                                     int32_t grid_h, int32_t grid_w, int32_t t0,
                                     float source_id, void* stream);

/* ------------------------------------------------------------------------
 * (Layer|RMS)Norm + AdaLN modulation.
 * Replaces joyomni_ops::fused_norm_scale_shift
 *   (deploy/joyomni_ops/csrc/fused_norm_scale_shift.cu:172-209; kernel :70-143).
 *   LN:  y = ((x - mu) * r * g + b) * (1 + scale) + shift,  r = 1/sqrt(var + eps)
 *   RMS: y = (x * r * g) * (1 + scale) + shift,            r = 1/sqrt(mean(x^2) + eps)
 * with fp32 arithmetic and one rounding to dtype. g = gamma (1 if NULL);
 * b = beta, used only by LN and only when gamma is given (0 otherwise), as in
 * the reference. x, y: [M, N] with row strides; scale, shift: [M, N] with row
 * strides (0 broadcasts a single [N] row to every row). N % 4 == 0.
 * ------------------------------------------------------------------------ */
int jo_fused_norm_scale_shift(const void* x, int64_t x_stride, const void* gamma,
                              const void* beta, const void* scale, int64_t scale_stride,
                              const void* shift, int64_t shift_stride, void* y,
                              int64_t y_stride, int64_t M, int64_t N, int dtype,
                              int norm_type, float eps, void* stream);

/* ------------------------------------------------------------------------
 * jo_fused_norm_scale_shift with per-sample modulation rows: scale and shift
 * row i serves rows [i * mod_rows, (i + 1) * mod_rows) of x (stride 0 still
 * broadcasts one row to all). The DiT's [B, D] AdaLN vectors over x
 * [B * L, D] are scale/shift with mod_rows = L, read in place — the
 * reference's caller (deploy/xvideo/models/dit/sgl_fused_ops.py:44-51)
 * expands them into [B * L, D] copies first. Same arithmetic and limits as
 * jo_fused_norm_scale_shift; mod_rows >= 1 (1 = a row each).
 * ------------------------------------------------------------------------ */
int jo_fused_norm_scale_shift_per_sample(const void* x, int64_t x_stride, const void* gamma,
                                         const void* beta, const void* scale,
                                         int64_t scale_stride, const void* shift,
                                         int64_t shift_stride, int64_t mod_rows, void* y,
                                         int64_t y_stride, int64_t M, int64_t N, int dtype,
                                         int norm_type, float eps, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm: out = (x * r) * w, r = 1/sqrt(mean(x^2) + eps), fp32 arithmetic.
 * Replaces joyomni_ops::rmsnorm (deploy/joyomni_ops/csrc/rmsnorm.cu:76-95;
 * kernel :37-61). x, out: [M, N] with row strides; weight: [N]. Any N >= 1.
 * ------------------------------------------------------------------------ */
int jo_rmsnorm(const void* x, int64_t x_stride, const void* weight, void* out,
               int64_t out_stride, int64_t M, int64_t N, int dtype, float eps,
               void* stream);

/* ------------------------------------------------------------------------
 * Per-head RMSNorm over rows read from a [tokens, heads, head_dim] view:
 * row (t, h) = x + t * x_token_stride + h * x_head_stride (elements), written
 * to out + (t * heads + h) * out_stride. r = 1/sqrt(mean(x^2) + eps).
 *   round_first == 0: out = (x * r) * w, one rounding — the caller
 *     rmsnorm_qk_bf16 (deploy/xvideo/models/dit/sgl_fused_ops.py:102-111)
 *     on the K slice of a packed qkv tensor, without its .contiguous() copy
 *     (:108); the same kernel and summation order as jo_rmsnorm.
 *   round_first == 1: out = round(round(x * r) * w), the torch RMSNorm
 *     module (deploy/xvideo/models/dit/dit.py:228-250, forward :247-249) as
 *     the text stream applies it to q and k (dit.py:384-385); the mean square
 *     is the exactly rounded mean of the exact squares.
 * head_dim >= 1; tokens * heads < 2^32.
 * ------------------------------------------------------------------------ */
int jo_rmsnorm_heads(const void* x, int64_t x_token_stride, int64_t x_head_stride,
                     const void* weight, void* out, int64_t out_stride, int64_t tokens,
                     int64_t heads, int64_t head_dim, int dtype, float eps, int round_first,
                     void* stream);

/* ------------------------------------------------------------------------
 * Residual add (optionally gated) + LayerNorm + AdaLN modulation, one pass:
 *   residual <- round(residual + x * gate)        (gate = 1 if NULL)
 *   y = LN(residual)(g, b) * (1 + scale) + shift  on the ROUNDED residual.
 * No reference counterpart: it fuses fused_add_gate / torch.addcmul
 *   (deploy/xvideo/models/dit/sgl_fused_ops.py:114-117) with the
 * fused_norm_scale_shift LayerNorm path (fused_norm_scale_shift.cu:88-142) as
 * the DiT block uses them back to back (dit.py:447-476).
 * x: [M, N]; residual: [M, N], updated in place; y: [M, N];
 * gate, scale, shift: row-strided, stride 0 = one [N] row for all; with a
 * nonzero stride, modulation row r serves rows r*mod_rows .. r*mod_rows +
 * mod_rows - 1 of x (mod_rows = 1: a row each; mod_rows = L: one row per
 * sample of a [B, L, N] batch, as the DiT's per-sample AdaLN vectors).
 * gamma/beta as in jo_fused_norm_scale_shift. N % 4 == 0.
 * ------------------------------------------------------------------------ */
int jo_fused_add_layernorm_scale_shift(const void* x, int64_t x_stride, void* residual,
                                       int64_t res_stride, const void* gate,
                                       int64_t gate_stride, const void* gamma,
                                       const void* beta, const void* scale,
                                       int64_t scale_stride, const void* shift,
                                       int64_t shift_stride, int64_t mod_rows, void* y,
                                       int64_t y_stride, int64_t M, int64_t N, int dtype,
                                       float eps, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm with an FP8 e4m3 quantization epilogue.
 *   v = (x * r) * w  in fp32 (never rounded to dtype), r as in jo_rmsnorm;
 *   group_size == 0:   one scale per row,       s: fp32 [M]
 *   group_size == 128: one scale per 1x128 block, s: fp32 [M, N/128] row-major
 *   s = amax(|v| over the group) / 448; q = e4m3fn_rne(clamp(v * inv, +-448)),
 *   inv = (s == 0) ? 0 : 1/s  — the per_token_quant_fp8 rule applied to v.
 * No reference counterpart: it fuses rmsnorm (rmsnorm.cu:41-60) with the
 * quantization of per_token_quant_fp8.cu:56-82 that Fp8Linear runs next
 * (deploy/xvideo/models/dit/fp8_linear.py:138-169).
 * x: [M, N] row-strided; out_q: fp8 [M, N] row stride q_stride.
 * N % 8 == 0, and N % 128 == 0 for group_size 128.
 * ------------------------------------------------------------------------ */
int jo_rmsnorm_quant_fp8(const void* x, int64_t x_stride, const void* weight, void* out_q,
                         int64_t q_stride, float* out_s, int64_t M, int64_t N, int dtype,
                         float eps, int64_t group_size, void* stream);

/* ------------------------------------------------------------------------
 * GELU (tanh approximation) + per-token FP8 e4m3 quantization of its output.
 * No reference counterpart: it fuses the MLP activation of the DiT block's
 * FP8 mode, torch.nn.functional.gelu(h, approximate="tanh")
 * (deploy/xvideo/models/dit/dit.py:91-92,433), with the activation
 * quantization of the following Fp8Linear.forward
 * (deploy/xvideo/models/dit/fp8_linear.py:140-166, per_token_quant_fp8.cu:56-82).
 *   a[r,j] = round_dtype(0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))), x = input[r,j]
 *     (fp32, tanh rounded to fp32 before the 1 is added, as the formula);
 *   then jo_sgl_per_token_quant_fp8's rule on the row a[r,:].
 * output_act (optional, may be NULL): the rounded activation a, row stride
 * act_stride; the FP8 bytes and scales are those of jo_sgl_per_token_quant_fp8
 * applied to it. output_act must not overlap input (JO_ERR_INVALID if the
 * byte ranges of the two views meet). Other arguments and limits as
 * jo_sgl_per_token_quant_fp8.
 * ------------------------------------------------------------------------ */
int jo_gelu_tanh_quant_fp8(const void* input, int dtype, int64_t num_tokens, int64_t hidden_dim,
                           int64_t in_stride, void* output_q, int64_t q_stride, float* output_s,
                           void* output_act, int64_t act_stride, void* stream);

/* ------------------------------------------------------------------------
 * (Gated residual add +) Layer|RMS norm + AdaLN, quantized per token to FP8
 * instead of written:
 *   residual <- round(residual + x * gate)   when residual != NULL (gate = 1
 *                                            if NULL), then v = residual;
 *   v = x                                    when residual == NULL;
 *   y = round_dtype(Norm(v)(g, b) * (1 + scale) + shift)   (never stored);
 *   s[m] = amax|y[m,:]| / 448; q = e4m3fn_rne(clamp(y * inv, +-448)),
 *   inv = (s == 0) ? 0 : 1/s.
 * Equal, byte for byte, to jo_fused_add_layernorm_scale_shift (or
 * jo_fused_norm_scale_shift) followed by jo_sgl_per_token_quant_fp8 on its y.
 * No reference counterpart: it fuses the DiT block's gated residual and
 * modulated norm (deploy/xvideo/models/dit/dit.py:447-476,
 * sgl_fused_ops.py:30-54,114-117, fused_norm_scale_shift.cu:88-142) with the
 * activation quantization Fp8Linear.forward runs on that y
 * (fp8_linear.py:138-169, per_token_quant_fp8.cu:56-82).
 * x: [M, N]; residual: [M, N] or NULL; gate, scale, shift: row-strided,
 * stride 0 = one [N] row for all, mod_rows consecutive rows of x per
 * modulation row otherwise (as in jo_fused_add_layernorm_scale_shift);
 * gamma/beta as in jo_fused_norm_scale_shift; out_q: fp8 [M, N] with row
 * stride q_stride; out_s: fp32 [M]. dtype bf16 or fp16; norm_type
 * JO_NORM_LAYER or JO_NORM_RMS; N % 4 == 0 and N > 0.
 * ------------------------------------------------------------------------ */
int jo_norm_scale_shift_quant_fp8(const void* x, int64_t x_stride, void* residual,
                                  int64_t res_stride, const void* gate, int64_t gate_stride,
                                  const void* gamma, const void* beta, const void* scale,
                                  int64_t scale_stride, const void* shift, int64_t shift_stride,
                                  int64_t mod_rows, void* out_q, int64_t q_stride, float* out_s,
                                  int64_t M, int64_t N, int dtype, int norm_type, float eps,
                                  void* stream);

/* ------------------------------------------------------------------------
 * Row-wise scaled FP8 GEMM with optional bias.
 * Replaces joyomni_ops::fp8_scaled_mm
 *   (deploy/joyomni_ops/csrc/fp8_gemm.cu:1450-1546; epilogue :99-136).
 *   acc[m, n] = sum_k A[m, k] * B[k, n]   (e4m3fn operands, fp32 accumulation)
 *   out[m, n] = round( scales_a[m] * (acc[m, n] * scales_b[n]) + bias[n] )
 * mat_a: fp8 [M, K] row-major, row stride lda bytes; mat_b: fp8 [K, N]
 * column-major (column n's K bytes contiguous), column stride ldb bytes;
 * scales_a fp32 [M]; scales_b fp32 [N]; bias [N] of out_dtype or NULL;
 * out: [M, N] row-major, row stride ldo elements, out_dtype BF16 or F16.
 * K % 16 == 0, N % 8 == 0, lda and ldb multiples of 16, operands 16-byte
 * aligned (the reference's alignment rules). K == 0 gives the epilogue of a
 * zero accumulator (the bias, or zeros) and reads no operand byte; mat_a and
 * mat_b may then be NULL.
 * ------------------------------------------------------------------------ */
int jo_fp8_scaled_mm(const void* mat_a, int64_t lda, const void* mat_b, int64_t ldb,
                     const float* scales_a, const float* scales_b, const void* bias, void* out,
                     int64_t ldo, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream);

/* jo_fp8_scaled_mm with a caller-owned device workspace (16-byte aligned).
 * With few output tiles and a long K (a few hundred rows: the text stream's
 * Fp8Linear calls, dit.py:59-92,381,438-444) the library may split K over
 * several workgroups per tile, which write fp32 partial products to the
 * workspace that a second kernel adds up in a fixed order: results are the
 * same on every run, and equal to jo_fp8_scaled_mm's up to fp32 summation
 * order. A workspace smaller than jo_fp8_scaled_mm_workspace_bytes(M, N, K)
 * (NULL with 0 bytes included) runs exactly as jo_fp8_scaled_mm. The
 * workspace is in use until the work queued on `stream` finishes; two calls
 * in flight at once need two workspaces. The torch op fp8_scaled_mm takes
 * it from the caching allocator. Reference counterpart: the same
 * fp8_scaled_mm (fp8_gemm.cu:1450-1546), whose CUTLASS kernel allocates its
 * own workspace. */
int jo_fp8_scaled_mm_ws(const void* mat_a, int64_t lda, const void* mat_b, int64_t ldb,
                        const float* scales_a, const float* scales_b, const void* bias, void* out,
                        int64_t ldo, int64_t M, int64_t N, int64_t K, int out_dtype,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes jo_fp8_scaled_mm_ws uses for an [M, K] x [K, N] product
 * under the current launch knobs: splits x M x N x 4, or 0 when it does not
 * split K (then no workspace is needed). A host-side computation. */
int64_t jo_fp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* jo_fp8_scaled_mm_ws without a caller workspace, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): no counterpart in the reference. The split-K partials
 * (jo_fp8_scaled_mm_workspace_bytes(M, N, K) bytes, the same plan as
 * jo_fp8_scaled_mm_ws with a workspace that size, so the same bits) go to a
 * static device array of 32 MiB that each GPU holds until the process ends;
 * a shape needing more is refused with JO_ERR_INVALID. It calls no
 * allocator. Every call on a GPU shares that GPU's array: two calls in
 * flight on one GPU at once (on two streams) race. */
int jo_fp8_scaled_mm_noalloc(const void* mat_a, int64_t lda, const void* mat_b, int64_t ldb,
                             const float* scales_a, const float* scales_b, const void* bias,
                             void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                             int out_dtype, void* stream);

/* ------------------------------------------------------------------------
 * RoPE'd K and copied V into a KV pool, every layer in one launch:
 *   dst_k[l, b, off + n, :] = apply_rotary_emb(src_k[l, b, n, :], cos[b, n], sin[b, n])
 *   dst_v[l, b, off + n, :] = src_v[l, b, n, :]           (when src_v != NULL)
 * with torch's evaluation of apply_rotary_emb (rope.py:21-28): per pair
 * (x0, x1) at columns (2i, 2i+1), out0 = fl(fl(x0*cos[2i]) - fl(x1*sin[2i])),
 * out1 = fl(fl(x1*cos[2i+1]) + fl(x0*sin[2i+1])) in fp32, then one rounding
 * to dtype — bit-identical to the reference for the same fp32 tables.
 * Replaces the per-layer loop of StreamingGraphRunner.run_commit
 * (deploy/xvideo/serving/graph_runner.py:137-142: 40 apply_rotary_emb + 80
 * copy kernels), its _seed_segment (:204-215) and, with layers = 1 and a
 * fresh destination, apply_rotary_emb itself (rope.py:21-28, used by
 * dit.py:211-217 and dit.py:384-385).
 * src: [layers, batch, tokens, num_heads * head_dim], dst: [layers, batch,
 * dst_tokens, num_heads * head_dim], with element strides (token rows
 * contiguous); dst_token_offset + tokens <= dst_tokens;
 * cos, sin: fp32 [batch?, tokens, head_dim] with token stride table_stride
 * and batch stride table_batch_stride (0 = one table for all batch rows).
 * dtype bf16 or fp16; head_dim even.
 * ------------------------------------------------------------------------ */
int jo_kv_commit_rope(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                      int64_t layers, int64_t batch, int64_t tokens, int64_t num_heads,
                      int64_t head_dim, int64_t src_layer_stride, int64_t src_batch_stride,
                      int64_t src_token_stride, int64_t dst_layer_stride,
                      int64_t dst_batch_stride, int64_t dst_token_stride,
                      int64_t dst_tokens, int64_t dst_token_offset, const float* cos,
                      const float* sin,
                      int64_t table_stride, int64_t table_batch_stride, int dtype,
                      void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* JOYOMNI_HIP_H */
