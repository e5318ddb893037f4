/*
 * walsh.h -- C ABI of libwalsh_hip.so, the MI355X (gfx950) implementation of
 * Walsh's ternary structured-linear hot path.
 *
 * Conventions (all entry points):
 *   - plain device pointers, int64 sizes/strides in elements, and a HIP
 *     stream passed as `void *` (a hipStream_t; NULL = the null stream);
 *   - work is enqueued on that stream; no entry point synchronises the host
 *     or allocates device memory;
 *   - return 0 on success, a negative WALSH_E* code for an invalid argument
 *     or unsupported shape (nothing is launched), or WALSH_EHIP when a HIP
 *     call fails; walsh_last_error() then returns a message (thread-local);
 *   - activations use `dtype` WALSH_F32 or WALSH_BF16 (inputs and outputs
 *     share it); parameters (alpha, beta, gamma, phi ...) are float32;
 *     arithmetic is float32 with float32 accumulation.
 *
 * Each declaration names the reference interface it replaces
 * (pulseofthemachine/Walsh-Research, file:line).
 */
#ifndef WALSH_H
#define WALSH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WALSH_ABI_VERSION 1

enum walsh_dtype { WALSH_F32 = 0, WALSH_BF16 = 1 };

enum walsh_status {
    WALSH_OK = 0,
    WALSH_EINVAL = -1,   /* bad pointer / size / stride */
    WALSH_ENOTSUP = -2,  /* shape or dtype this build does not handle */
    WALSH_EHIP = -3      /* a HIP runtime call failed */
};

/* Library identity and errors. */
int walsh_abi_version(void);
const char *walsh_last_error(void);
/* Binary name of the device code this library carries ("gfx950"). */
const char *walsh_device_arch(void);

/* Kernel timing -- a measurement hook with no counterpart in the reference,
 * for callers that report per-kernel time (benchmarks, profilers).
 * walsh_timing_begin(capacity): from now on every kernel launch records its
 *   own start/stop timestamps (hipExtLaunchKernelGGL) into the next of
 *   `capacity` event pairs, labelled with the tag last set by
 *   walsh_timing_tag (initially -1).  Launches beyond capacity are untimed.
 * walsh_timing_end(tags, ms, capacity): stops timing, waits for the timed
 *   kernels and writes up to `capacity` (tag, milliseconds) pairs in launch
 *   order; returns how many were written (negative on error).
 * Not thread-safe while timing is on. */
int walsh_timing_begin(int capacity);
void walsh_timing_tag(int tag);
int walsh_timing_end(int *tags, float *ms, int capacity);

/* ------------------------------------------------------------------ A1 / A11
 * Absmean ternary quantisation.
 * Replaces TernaryAbsmeanSTE.forward / quantize_ternary
 *   (src/model/physics.py:21-51) and the MoE variant
 *   (src/model/moe.py:276-303).
 *
 * walsh_ternary_gamma: gamma = mean(|w|) + 1e-8 (float32) over n weights,
 *   reduced deterministically in float64 by one workgroup (same result on
 *   every call and every device).  Writes one float to *gamma.
 */
int walsh_ternary_gamma(const float *w, int64_t n, float *gamma, void *stream);

/* walsh_ternary_quantize: codes = clamp(round_half_even(w / *gamma), -1, 1)
 *   for w viewed as [rows, K] (row-major, contiguous).  Any output may be
 *   NULL:
 *     codes  int8  [rows, K]
 *     packed uint8 [rows, ceil(K/4)] in the 2-bit layout of
 *            pack_ternary_weights (src/model/fht_cuda.py:65-93):
 *            byte = v0<<6 | v1<<4 | v2<<2 | v3, v = code + 1; K is padded
 *            to a multiple of 4 with code 0;
 *     scaled float [rows, K] = code * gamma (the MoE quantiser's value,
 *            src/model/moe.py:288).
 *   `gamma` is a device pointer (usually walsh_ternary_gamma's output).
 */
int walsh_ternary_quantize(const float *w, int64_t rows, int64_t K, const float *gamma,
                           int8_t *codes, uint8_t *packed, float *scaled, void *stream);

/* walsh_ternary_ste_bwd: backward of the two straight-through estimators,
 *   elementwise over n float32 gradients (out may alias grad):
 *   mode 0, TernaryAbsmeanSTE of src/model/physics.py:13-50 as used through
 *     quantize_ternary (w_clamped + (w_quant - w_clamped).detach()):
 *     out = grad where -1.5 <= w <= 1.5, else 0 (w: the latent weights);
 *   mode 1, TernaryAbsmeanSTE.backward of src/model/moe.py:289-294:
 *     out = clamp(grad, -2, 2) (w unused, may be NULL). */
int walsh_ternary_ste_bwd(const float *grad, const float *w, int64_t n, int mode, float *out, void *stream);

/* walsh_bitmask_workspace_bytes / walsh_ternary_from_bitmask: decode the
 *   .walsh v4 bitmask + sign storage of a ternary tensor (written by
 *   compress.py:36-93, read by generate_compressed.py:70-105) on the GPU,
 *   straight into the 2-bit packed layout and/or int8 codes of the tensor
 *   viewed as [rows, K] (K = last dim):
 *     bitmask: bit p (LSB first) set <=> value p is non-zero;
 *     sign_bits: bit r set <=> the r-th non-zero is +1 (clear: -1);
 *   non-zeros past num_nonzero decode as 0, as the reference loader leaves
 *   them.  rows*K < 2^32; workspace: walsh_bitmask_workspace_bytes(rows*K). */
int64_t walsh_bitmask_workspace_bytes(int64_t total);
int walsh_ternary_from_bitmask(const uint8_t *bitmask, int64_t bitmask_bytes, const uint8_t *sign_bits,
                               int64_t sign_bytes, int64_t num_nonzero, int64_t rows, int64_t K, uint8_t *packed,
                               int8_t *codes, void *workspace, int64_t workspace_bytes, void *stream);

/* walsh_ternary_unpack: inverse of the packed layout -> int8 codes [rows, K]
 *   (unpack_ternary_weights, src/model/fht_cuda.py:96-117). */
int walsh_ternary_unpack(const uint8_t *packed, int64_t rows, int64_t K, int8_t *codes,
                         void *stream);

/* ------------------------------------------------------------------ A3-A6
 * Hadamard-32 ternary linear forward.
 * Replaces HadamardLinear.forward (src/model/fht_cuda.py:489-519), which is
 * also what HadamardTernaryLinearTuple (:550-569) and HadamardTernaryLinear
 * (:392-424) compute:
 *   x row (32*in_o) viewed [32 g][in_o i];
 *   y[h, o] = beta[h, o] * sum_g H[g, h] sum_i W[g, o, i] sum_g' H[g', g] alpha[g', i] x[g', i]
 *   with H the normalised Sylvester matrix (fht_cuda.py:32-56).
 *
 * walsh_hadamard_weight_bytes: size of the kernel weight layout for a shape.
 * walsh_hadamard_prepare: reorders 2-bit packed codes [32, out_o, ceil(in_o/4)]
 *   (walsh_ternary_quantize's `packed`) into that layout.  Call once per
 *   weight version; the layout holds the same bytes, permuted.
 */
int64_t walsh_hadamard_weight_bytes(int64_t in_o, int64_t out_o);
int walsh_hadamard_prepare(const uint8_t *packed, int64_t in_o, int64_t out_o,
                           uint8_t *kweight, void *stream);

/* walsh_hadamard_linear_fwd: y[M, ldy] = layer(x[M, ldx]).
 *   x row m starts at x + m*ldx (elements); only the first 32*in_o entries
 *   are read; y row m's first 32*out_o entries are written.
 *   alpha float [32, in_o]; beta float [32, out_o]; kweight from
 *   walsh_hadamard_prepare.  dtype: WALSH_F32 (float32 matrix cores) or
 *   WALSH_BF16 (bf16 matrix cores on bf16-rounded transformed activations,
 *   float32 accumulation). */
int walsh_hadamard_linear_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                              const uint8_t *kweight, const float *alpha, const float *beta,
                              void *y, int64_t ldy, int dtype, void *stream);

/* walsh_hadamard_linear_ex_fwd: walsh_hadamard_linear_fwd with explicit group
 *   strides: x row element (g, i) at g*gsx + i (gsx >= in_o), y row element
 *   (h, o) at h*gsy + o (gsy >= out_o).  With gsy > out_o the slots o in
 *   [out_o, roundup(out_o, 4)) are written as exact zeros; slots i in
 *   [in_o, gsx) of x must hold finite values (they meet zero weights).  Used
 *   for the group-padded SwiGLU hidden layout (see walsh_hadamard_swiglu_fwd). */
int walsh_hadamard_linear_ex_fwd(const void *x, int64_t ldx, int64_t gsx, int64_t M, int64_t in_o, int64_t out_o,
                                 const uint8_t *kweight, const float *alpha, const float *beta, void *y, int64_t ldy,
                                 int64_t gsy, int dtype, void *stream);

/* walsh_hadamard_linear_rope_fwd: walsh_hadamard_linear_fwd followed by
 *   apply_rotary_emb (src/model/chassis.py:339-345) on its output, in the
 *   store: output row r is token t = r % rope_T of a sequence, split into
 *   heads of head_dim features whose pairs (2i, 2i+1) turn by rope[t][i] =
 *   (cos, sin) (float32 [rope_T][head_dim/2][2], the view_as_real of the
 *   freqs_cis rows of the call).  head_dim % 4 == 0 and divides out_o; rows
 *   and in_o 4-aligned.  Used for the q and k projections. */
int walsh_hadamard_linear_rope_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                   const uint8_t *kweight, const float *alpha, const float *beta, const float *rope,
                                   int64_t rope_T, int64_t head_dim, void *y, int64_t ldy, int dtype, void *stream);

/* walsh_hadamard_linear_multi_fwd: n (<= 4) Hadamard linears of one shape on
 *   the same input rows x, in one launch where the shape allows (the q, k and
 *   v projections of CausalSelfAttention.forward, chassis.py:441-452): layer i
 *   uses kweights[i], alphas[i], betas[i] and writes ys[i] (row stride ldy);
 *   layers with bit i of rope_mask also apply the rotary embedding of
 *   walsh_hadamard_linear_rope_fwd (rope, rope_T, head_dim).  Shapes the
 *   single-tile kernel does not take run as n launches. */
int walsh_hadamard_linear_multi_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o, int64_t n,
                                    const uint8_t *const *kweights, const float *const *alphas,
                                    const float *const *betas, void *const *ys, int64_t ldy, const float *rope,
                                    int64_t rope_T, int64_t head_dim, int rope_mask, int dtype, void *stream);

/* walsh_hadamard_linear_multi_ex_fwd: walsh_hadamard_linear_multi_fwd with
 *   each output's own row stride ldys[i] and group stride gsys[i]
 *   (element (row, g, o) of output i at ys[i] + row*ldys[i] + g*gsys[i] + o;
 *   gsys[i] >= out_o, ldys[i] >= 32*gsys[i]): lets the k and v projections
 *   of a decode step write straight into a head-major KV cache slot
 *   ([batch][head][position][head_dim], CausalSelfAttention.forward with
 *   KVCache.update, chassis.py:441-455). */
int walsh_hadamard_linear_multi_ex_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                       int64_t n, const uint8_t *const *kweights, const float *const *alphas,
                                       const float *const *betas, void *const *ys, const int64_t *ldys,
                                       const int64_t *gsys, const float *rope, int64_t rope_T, int64_t head_dim,
                                       int rope_mask, int dtype, void *stream);

/* walsh_hadamard_swiglu_fwd: h = silu(gate(x)) * up(x) for two Hadamard
 *   linears of the same shape (in_o -> hid_o) on the same input, fused
 *   (SwiGLUMLP.forward, src/model/chassis.py:498-504, gate_proj/up_proj).
 *   h is written with group stride gsh (>= hid_o; pad slots up to
 *   roundup(hid_o, 4) get zeros), ready for down_proj through
 *   walsh_hadamard_linear_ex_fwd with gsx = gsh. */
int walsh_hadamard_swiglu_fwd(const void *x, int64_t ldx, int64_t gsx, int64_t M, int64_t in_o, int64_t hid_o,
                              const uint8_t *kw_gate, const float *alpha_gate, const float *beta_gate,
                              const uint8_t *kw_up, const float *alpha_up, const float *beta_up, void *h,
                              int64_t ldh, int64_t gsh, int dtype, void *stream);

/* walsh_hadamard_mlp_fwd: the whole SwiGLUMLP.forward, down(silu(gate(x)) *
 *   up(x)) (src/model/chassis.py:498-504), in one launch for bf16 rows with
 *   gate/up in_o -> hid_o and down hid_o -> out_o, in_o and out_o <= 16
 *   (multiples of 4, e.g. n_embd 512) and 16 < hid_o <= 48 (two or three
 *   16-wide hidden tiles).  x rows of 32*in_o values at x + m*ldx, y rows of
 *   32*out_o at y + m*ldy; weights from walsh_hadamard_prepare for each
 *   shape.  The hidden activation stays on chip; the result equals
 *   walsh_hadamard_swiglu_fwd (gsh = roundup(hid_o, 4)) followed by
 *   walsh_hadamard_linear_ex_fwd of the down projection bitwise. */
int walsh_hadamard_mlp_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t hid_o, int64_t out_o,
                           const uint8_t *kw_gate, const float *alpha_gate, const float *beta_gate,
                           const uint8_t *kw_up, const float *alpha_up, const float *beta_up,
                           const uint8_t *kw_down, const float *alpha_down, const float *beta_down, void *y,
                           int64_t ldy, int dtype, void *stream);

/* walsh_hadamard_dense_weight_bytes / walsh_hadamard_dense_prepare: float32
 *   weights of a Hadamard-structured layer with dense per-group matrices
 *   (HadamardHeadMixerFused.W [32, head_dim, head_dim], fht_cuda.py:627-648)
 *   in the kernel's matrix-core layout, bf16 or float32 (dtype).  w is
 *   [32][out_o][in_o], or [32][in_o][out_o] when w_io (the head mixer's
 *   x @ W[h]).  Re-run after every weight update. */
int64_t walsh_hadamard_dense_weight_bytes(int64_t in_o, int64_t out_o, int dtype);
int walsh_hadamard_dense_prepare(const float *w, int64_t in_o, int64_t out_o, int w_io, int dtype, uint8_t *kweight,
                                 void *stream);

/* walsh_head_mixer_fwd: HadamardHeadMixerFused.forward (fht_cuda.py:650-662)
 *   on one group of 32 attention heads: x element (b, h, t, d) at
 *   b*x_bstride + h*x_hstride + t*x_tstride + d (the [B, 32, T, D] output of
 *   scaled_dot_product_attention, or a view into more heads); the result is
 *   written token-major, y row b*T + t at (b*T + t)*ldy holding head h at
 *   h*D: the layout the output projection reads, so no transpose copy is
 *   needed.  y = beta[d] * H (H x W[h]) over the head axis, H the normalised
 *   32-point Hadamard matrix.  kweight from walsh_hadamard_dense_prepare with
 *   w_io = 1 and the same dtype.  head_dim (D) <= 32, or, in bf16,
 *   D <= 128 with 4-aligned strides (the wide kernel streams the weights). */
int walsh_head_mixer_fwd(const void *x, int64_t B, int64_t T, int64_t D, int64_t x_bstride, int64_t x_hstride,
                         int64_t x_tstride, const uint8_t *kweight, const float *beta, void *y, int64_t ldy, int dtype,
                         void *stream);

/* walsh_head_mixer_proj_fwd: the attention block's head mixer followed by
 *   its output projection (chassis.py:465-478: HadamardHeadMixerFused.forward,
 *   fht_cuda.py:650-662, then self.wo, HadamardLinear.forward,
 *   fht_cuda.py:489-519) in one launch, for head_dim 16, one group of 32
 *   heads and a 16x16 projection, bf16.  x as in walsh_head_mixer_fwd; the
 *   mixer's output rows are rounded to bf16 as walsh_head_mixer_fwd stores
 *   them and go straight into the projection (mix_kweight from
 *   walsh_hadamard_dense_prepare with w_io = 1, proj_kweight from
 *   walsh_hadamard_prepare; proj_alpha may be NULL for all ones); y row
 *   b*T + t at (b*T + t)*ldy, 512 values.  The result equals
 *   walsh_head_mixer_fwd then walsh_hadamard_linear_fwd bitwise. */
int walsh_head_mixer_proj_fwd(const void *x, int64_t B, int64_t T, int64_t x_bstride, int64_t x_hstride,
                              int64_t x_tstride, const uint8_t *mix_kweight, const float *mix_beta,
                              const uint8_t *proj_kweight, const float *proj_alpha, const float *proj_beta, void *y,
                              int64_t ldy, int dtype, void *stream);

/* ------------------------------------------------------------------ backward
 * Autograd of HadamardLinear.forward (src/model/fht_cuda.py:489-519) through
 * FHTFunction.backward (fht_cuda.py:328-332, H self-adjoint) and the
 * straight-through estimator of physics.quantize_ternary
 * (src/model/physics.py:43-50): replaces the torch autograd graph the
 * reference builds for the layer.
 *
 * walsh_hadamard_pack_transpose: the reference 2-bit packing (fht_cuda.py:
 *   65-93) of the transposed codes, packed_t [32][in_o][ceil(out_o/4)] from
 *   packed [32][out_o][ceil(in_o/4)].  walsh_hadamard_prepare(packed_t,
 *   out_o, in_o, kweight_t) then gives the transposed layer's kernel layout.
 * walsh_hadamard_bwd_workspace_bytes: device scratch walsh_hadamard_linear_bwd
 *   needs for M dense rows (row strides 32*in_o / 32*out_o).
 * walsh_hadamard_linear_bwd: for the output gradient gy [M, ldg] of
 *   y = beta .* H W H (alpha .* x), x [M, ldx]:
 *     gx     = alpha .* H W^T H (beta .* gy)          [M, ldgx], x's dtype
 *     dalpha = sum_rows x .* H W^T H (beta .* gy)      float [32][in_o]
 *     dbeta  = sum_rows gy .* H W H (alpha .* x)       float [32][out_o]
 *     dweight = sum_rows H(beta .* gy)_g (x) H(alpha .* x)_g, times
 *              [-1.5 <= latent <= 1.5] when latent (float [32][out_o][in_o])
 *              is given (the STE's clamp): float [32][out_o][in_o]
 *   Any of gx / dalpha / dbeta / dweight may be null (not computed).
 *   kweight (forward layout) is needed for dbeta, kweight_t for gx / dalpha.
 *   Sums run in a fixed order (identical results run to run).  The outputs
 *   are overwritten, not accumulated. */
int walsh_hadamard_pack_transpose(const uint8_t *packed, int64_t in_o, int64_t out_o, uint8_t *packed_t,
                                  void *stream);
int64_t walsh_hadamard_bwd_workspace_bytes(int64_t M, int64_t in_o, int64_t out_o, int dtype);
int walsh_hadamard_linear_bwd(const void *x, int64_t ldx, const void *gy, int64_t ldg, int64_t M, int64_t in_o,
                              int64_t out_o, const uint8_t *kweight, const uint8_t *kweight_t, const float *alpha,
                              const float *beta, const float *latent, void *gx, int64_t ldgx, float *dalpha,
                              float *dbeta, float *dweight, int dtype, void *workspace, int64_t workspace_bytes,
                              void *stream);
/* walsh_hadamard_linear_ex_bwd: walsh_hadamard_linear_bwd with the group
 *   strides of walsh_hadamard_linear_ex_fwd: x and gx rows hold group g at
 *   g*gsx (gsx >= in_o), gy rows at g*gsy (gsy >= out_o); gx slots in
 *   [in_o, roundup(in_o, 4)) are written as zeros (slots past that are not
 *   written), pad slots of x and gy are not read.  The backward of the
 *   group-padded SwiGLU hidden layout. */
int walsh_hadamard_linear_ex_bwd(const void *x, int64_t ldx, int64_t gsx, const void *gy, int64_t ldg, int64_t gsy,
                                 int64_t M, int64_t in_o, int64_t out_o, const uint8_t *kweight,
                                 const uint8_t *kweight_t, const float *alpha, const float *beta, const float *latent,
                                 void *gx, int64_t ldgx, float *dalpha, float *dbeta, float *dweight, int dtype,
                                 void *workspace, int64_t workspace_bytes, void *stream);

/* walsh_fht_fwd: fast Walsh-Hadamard transform of `rows` contiguous rows of
 *   length n (power of two <= 16384), Sylvester order, scaled by 1/sqrt(n)
 *   when `normalize` (fht_butterfly / fht, src/model/fht_cuda.py:281-337). */
int walsh_fht_fwd(const void *x, int64_t rows, int64_t n, int normalize, void *y, int dtype, void *stream);

/* ------------------------------------------------------------------ A7-A9
 * Octonion (Cayley-Dickson) ternary linear forward.
 * Replaces OctonionTernaryLinearRef.forward (src/model/physics.py:66-82) and
 * OctonionFusedLinear -> cayley_dickson_fused -> cayley_dickson_fused_kernel
 * (src/model/cayley_dickson_cuda.py:650-668, :574-619, :313-421):
 *   y_i = beta * sum_j S[i][j] x_j W[i^j]^T, parts x_j = x[:, j*in_o:(j+1)*in_o]
 *   and y_i = y[:, i*out_o:(i+1)*out_o], S = SIGN_TABLE (constants.py:13-31).
 *
 * walsh_octonion_weight_elems: element count of the expanded block matrix
 *   B [8*out_o, Kp], Kp = roundup(8*in_o, 32).
 * walsh_octonion_prepare: B[i*out_o + n][j*in_o + k] = S[i][j] * W[i^j][n][k]
 *   from packed codes [8, out_o, ceil(in_o/4)]; dtype = element type of B
 *   (use the activation dtype).  Once per weight version.
 * walsh_octonion_linear_fwd: y[M, ldy] = (x[M, ldx] B^T) * beta[n % out_o];
 *   beta float [out_o]; x rows 16-byte aligned.  WALSH_BF16 multiplies bf16
 *   operands (the reference's kernel casts x to bf16 too, :402) with float32
 *   accumulation and stores bf16(x B^T * beta), one rounding: within one
 *   bf16 ulp of bf16(walsh_octonion_fused_fwd's float32 output), the value
 *   the reference's next layer reads after its bf16 cast, so a stack of
 *   layers chains this output; WALSH_F32 uses float32 matrix cores.  beta
 *   may be null (all ones).
 *
 * Backward (CayleyDicksonFunction.backward, src/model/cayley_dickson_cuda.py:
 * 500-567, with physics.quantize_ternary's STE, physics.py:43-50):
 * walsh_octonion_prepare_t: Bt[j*in_o + m][i*out_o + n] = S[i][j] *
 *   W[i^j][n][m] * beta[n], rows of length roundup(8*out_o, 32); then
 *   gx = walsh_octonion_linear_fwd(gy, in_o' = out_o, out_o' = in_o, Bt,
 *   beta = null) is the input gradient (gy .* beta) B.
 * walsh_octonion_bwd_fold: parameter gradients from C = gy^T x (float
 *   [8*out_o][ldc], the sum of n_parts partial matrices part_stride floats
 *   apart, e.g. split-K results of any GEMM):
 *     dweight[w][n][m] = beta[n] sum_i S[i][i^w] C[i*out_o + n][(i^w)*in_o + m],
 *       zeroed where latent (float [8][out_o][in_o], optional) is outside
 *       [-1.5, 1.5];
 *     dbeta[n] = sum_{i,j,m} S[i][j] W[i^j][n][m] C[i*out_o + n][j*in_o + m].
 *   Either output may be null.  Fixed-order sums (float64). */
int64_t walsh_octonion_weight_elems(int64_t in_o, int64_t out_o);
int walsh_octonion_prepare(const uint8_t *packed, int64_t in_o, int64_t out_o, void *B, int dtype, void *stream);
int walsh_octonion_linear_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o, const void *B,
                              const float *beta, void *y, int64_t ldy, int dtype, void *stream);
int walsh_octonion_prepare_t(const uint8_t *packed, int64_t in_o, int64_t out_o, const float *beta, void *Bt,
                             int dtype, void *stream);

/* walsh_octonion_fused_fwd: the reference module's forward and output dtype,
 *   OctonionFusedLinear.forward / OctonionPackedLinear.forward
 *   (src/model/cayley_dickson_cuda.py:650-668, :761-765): the fused kernel
 *   multiplies bf16 x by the bf16 weights with float32 accumulation and
 *   returns bf16 (:402, :411, :421); the module then multiplies by the float32
 *   beta, which promotes to float32.  Here:
 *     y[M, ldy] (float32) = float(bf16(x B^T)) * beta[n % out_o],
 *   x bf16 [M, ldx] (a float32 input is rounded to bf16 by the caller, as the
 *   reference kernel does at :402), B from walsh_octonion_prepare in bf16,
 *   beta float [out_o] or null (ones).  Rows of x, B and y 16-byte aligned. */
int walsh_octonion_fused_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o, const void *B,
                             const float *beta, float *y, int64_t ldy, void *stream);
int walsh_octonion_bwd_fold(const float *C, int64_t ldc, int64_t n_parts, int64_t part_stride, const uint8_t *packed,
                            int64_t in_o, int64_t out_o, const float *beta, const float *latent, float *dweight,
                            float *dbeta, void *stream);

/* walsh_octonion_bwd_params: the parameter gradients of
 *   walsh_octonion_bwd_fold with C = gy^T x formed here, on the GPU:
 *   gy [M, ldg] and x [M, ldx] (dtype) are transposed into token-contiguous
 *   rows in the workspace, a split-K matrix-core GEMM writes float32 partial
 *   sums of C (one per K split) and the fold adds them in split order
 *   (the dW kernel of cayley_dickson_cuda.py:225-307 with the dbeta sum of
 *   :540-563).  work: walsh_octonion_bwd_params_workspace_bytes(M, in_o,
 *   out_o, dtype) bytes, 256-byte aligned.  M >= 1. */
int64_t walsh_octonion_bwd_params_workspace_bytes(int64_t M, int64_t in_o, int64_t out_o, int dtype);
int walsh_octonion_bwd_params(const void *gy, int64_t ldg, const void *x, int64_t ldx, int64_t M, int64_t in_o,
                              int64_t out_o, const uint8_t *packed, const float *beta, const float *latent,
                              float *dweight, float *dbeta, int dtype, void *work, int64_t work_bytes, void *stream);

/* ------------------------------------------------------------------ decode attention
 * CausalSelfAttention.forward with a KV cache at T == 1
 * (src/model/chassis.py:441-478, cache :262-330): o = softmax(q K^T * scale) V
 * over the L cached positions, no mask.
 *
 * walsh_decode_attention_workspace_bytes: float scratch for the split-K
 *   partials of one call.
 * walsh_decode_attention: q element (b, h, d) at b*q_bs + h*q_hs + d; cache
 *   element (b, h, j, d) at b*kv_bs + h*kv_hs + j*kv_rs + d for k and v (the
 *   KV cache's [batch, n_head, max_seq_len, head_dim] storage); o element
 *   (b, h, d) at b*o_bs + h*o_hs + d.  head_dim D in {16, 32, 64, 128};
 *   strides multiples of 8 elements, q / k / v 16-byte aligned.  dtype is
 *   that of q, k, v and o; scores, softmax and sums in float32. */
int64_t walsh_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t D);
int walsh_decode_attention(const void *q, int64_t q_bs, int64_t q_hs, const void *k, const void *v, int64_t kv_bs,
                           int64_t kv_hs, int64_t kv_rs, int64_t B, int64_t H, int64_t L, int64_t D, float scale,
                           void *o, int64_t o_bs, int64_t o_hs, int dtype, void *workspace, int64_t workspace_bytes,
                           void *stream);

/* walsh_decode_attention_static: walsh_decode_attention without the
 *   workspace; it allocates nothing.  No counterpart in the reference: it is
 *   for callers that cannot allocate device memory (code under HIP graph
 *   capture, serving loops, harnesses that forbid hipMalloc).  The split-K
 *   partials live in a file-scope device array of the library, 8 MiB per GPU
 *   (held until the process ends); a call whose partials need more
 *   (B * H * S * (D + 2) * 4 bytes, the size walsh_decode_attention_workspace_bytes
 *   reports) returns WALSH_ENOTSUP without launching.  Every call on one GPU
 *   shares that GPU's array: calls that overlap on one GPU (other streams or
 *   host threads) race and must be serialised by the caller.  Same arguments,
 *   layouts and results as walsh_decode_attention (the same kernels). */
int walsh_decode_attention_static(const void *q, int64_t q_bs, int64_t q_hs, const void *k, const void *v,
                                  int64_t kv_bs, int64_t kv_hs, int64_t kv_rs, int64_t B, int64_t H, int64_t L,
                                  int64_t D, float scale, void *o, int64_t o_bs, int64_t o_hs, int dtype,
                                  void *stream);

/* walsh_prefill_attention: causal self-attention of T queries against the
 *   same T keys per (sequence, head), F.scaled_dot_product_attention(q, k,
 *   v, is_causal=True) of CausalSelfAttention.forward without a cache
 *   (src/model/chassis.py:465): o = softmax(q k^T * scale, key <= query) v.
 *   Element (b, h, t, d) of q at b*q_sb + h*q_sh + t*q_st + d, of k and v at
 *   b*kv_sb + h*kv_sh + t*kv_st + d, of o at b*o_sb + h*o_sh + t*o_st + d
 *   (any of the [B, T, H, D] or [B, H, T, D] layouts).  bf16 only; head_dim
 *   D in {16, 32, 64, 128}; strides multiples of 8 elements, pointers
 *   16-byte aligned.  Scores, softmax and sums in float32, the
 *   probabilities rounded to bf16 for the product with v. */
int walsh_prefill_attention(const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void *k, const void *v,
                            int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t B, int64_t H, int64_t T, int64_t D,
                            float scale, void *o, int64_t o_sb, int64_t o_sh, int64_t o_st, int dtype, void *stream);

/* ------------------------------------------------------------------ A14-A17
 * mHC residual streams.  Stream tensors are [M tokens][n streams][C] with row
 * stride ldx >= n*C (elements); n <= 4 and C % 4 == 0 in this build.
 *
 * walsh_sinkhorn_fwd: SinkhornKnopp.forward / sinkhorn_knopp_fused
 *   (src/model/mhc.py:214-229, :152-195): out = n_iter x {column-normalise,
 *   row-normalise}(exp(h)) with `eps` added to every sum; h, out float32
 *   [batch, n, n], n <= 8.
 */
int walsh_sinkhorn_fwd(const float *h, int64_t batch, int64_t n, int64_t n_iter, float eps, float *out,
                       void *stream);

/* walsh_sinkhorn_bwd: gradient of walsh_sinkhorn_fwd (the autograd torch
 *   derives for SinkhornKnopp.forward, src/model/mhc.py:214-229): dh = the
 *   gradient wrt h for the output gradient g, float32 [batch, n, n], n <= 8.
 *   The forward's intermediates are recomputed bit-identically per iteration
 *   (O(n_iter^2) small steps per matrix), so nothing is saved between passes. */
int walsh_sinkhorn_bwd(const float *h, const float *g, int64_t batch, int64_t n, int64_t n_iter, float eps, float *dh,
                       void *stream);

/* walsh_mhc_pre_fwd: the three ResidualStreamMapping.forward calls of one
 *   mHCResidualStream.forward and its H_pre @ x (src/model/mhc.py:283-318,
 *   :345-364), fused.  With x_hat = x / sqrt(mean(x^2) + rms_eps) over the
 *   n*C row and dyn = phi . x_hat:
 *     h_pre  [M, n]    = sigmoid(coef[0]*dyn[0:n] + bias[0:n])
 *     h_post [M, n]    = 2*sigmoid(coef[1]*dyn[n:2n] + bias[n:2n])
 *     h_res  [M, n, n] = Sinkhorn(coef[2]*dyn[2n:2n+n*n] + bias[2n:], n_iter, sk_eps)
 *     layer_in [M, C]  = sum_s h_pre[:, s] * x[:, s, :]   (row stride ld_in)
 *   phi: activation dtype, [32, n*C] rows = phi_pre (n), phi_post (n),
 *   phi_res (n*n), zero rows to 32.  coef = alphas (pre, post, res); bias =
 *   float32 [2n + n*n].  rms_eps is finfo(activation dtype).eps in the
 *   reference (F.rms_norm with eps=None, mhc.py:291). */
int walsh_mhc_pre_fwd(const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C, const void *phi,
                      const float *coef, const float *bias, float rms_eps, int64_t n_iter, float sk_eps,
                      float *h_pre, float *h_post, float *h_res, void *layer_in, int64_t ld_in, int dtype,
                      void *stream);

/* walsh_mhc_pre_norm_fwd: walsh_mhc_pre_fwd for rows of up to 8 KB (n*C*esize
 *   <= 8192, C <= 1024, n*C % 16 == 0), each workgroup keeping its token tile
 *   in LDS so x is read once; phi_frag is phi in matrix-core fragment order
 *   [n*C/16][2][64][4] (element (ks, nt, lane = 16*kq + r, j) =
 *   phi[16*nt + r][16*ks + 4*kq + j]).  If norm_w is non-NULL, layer_in is
 *   also RMS-normalised over its C values and scaled by norm_w (float32 [C]):
 *   layer_in * rsqrt(mean(layer_in^2) + norm_eps) * norm_w, the block's
 *   attention_norm / ffn_norm (src/model/chassis.py:96-106) fused in. */
int walsh_mhc_pre_norm_fwd(const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C, const void *phi_frag,
                           const float *coef, const float *bias, float rms_eps, int64_t n_iter, float sk_eps,
                           float *h_pre, float *h_post, float *h_res, void *layer_in, int64_t ld_in,
                           const float *norm_w, float norm_eps, int dtype, void *stream);

/* walsh_mhc_post_pre_norm_fwd: the stream update of one mHCResidualStream
 *   (src/model/mhc.py:366-381) fused with the mappings of the next one
 *   (walsh_mhc_pre_norm_fwd): the tile of the next stream's input
 *     x_new[t, r, :] = sum_s h_res_prev[t, r, s] x_old[t, s, :] + h_post_prev[t, r] out[t, :]
 *   is formed while it is loaded (x_old read once, the separate pre pass's
 *   read of x_new saved), written to x_new (row stride ld_new) and used for
 *   h_pre / h_post / h_res / layer_in exactly as walsh_mhc_pre_norm_fwd uses
 *   x.  x_new is bitwise what walsh_mhc_post_fwd writes.  Same limits as
 *   walsh_mhc_pre_norm_fwd, plus C*esize % 16 == 0 and 16-byte aligned rows;
 *   x_new may not alias x_old, nor the new h_post / h_res the previous ones. */
int walsh_mhc_post_pre_norm_fwd(const void *x_old, int64_t ld_old, const void *out, int64_t ld_out,
                                const float *h_res_prev, const float *h_post_prev, void *x_new, int64_t ld_new,
                                int64_t M, int64_t n, int64_t C, const void *phi_frag, const float *coef,
                                const float *bias, float rms_eps, int64_t n_iter, float sk_eps, float *h_pre,
                                float *h_post, float *h_res, void *layer_in, int64_t ld_in, const float *norm_w,
                                float norm_eps, int dtype, void *stream);

/* walsh_mhc_pre_wide_fwd: the same results as walsh_mhc_pre_norm_fwd for
 *   rows too long for an LDS tile (n*C % 32 == 0, C <= 4096; n_embd 4096),
 *   in two launches: a split-K projection on 16x16x32 matrix cores writing
 *   partial sums to `workspace`, then per token the constraints and
 *   layer_in (with its RMSNorm when norm_w is given).  phi_frag32 is the
 *   [32, n*C] projection in fragment order [n*C/32][2][64][8] (lane
 *   16*kq + r holds phi[16*tile + r][32*ks + 8*kq .. +7]).  workspace:
 *   device memory of at least walsh_mhc_pre_wide_workspace(M, n, C) bytes. */
int64_t walsh_mhc_pre_wide_workspace(int64_t M, int64_t n, int64_t C);
int walsh_mhc_pre_wide_fwd(const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C, const void *phi_frag32,
                           const float *coef, const float *bias, float rms_eps, int64_t n_iter, float sk_eps,
                           float *h_pre, float *h_post, float *h_res, void *layer_in, int64_t ld_in,
                           const float *norm_w, float norm_eps, void *workspace, int64_t workspace_bytes, int dtype,
                           void *stream);

/* walsh_mhc_post_pre_wide_fwd: the stream update of one mHCResidualStream
 *   (src/model/mhc.py:366-381) fused with the wide mappings of the next one
 *   (walsh_mhc_pre_wide_fwd, src/model/mhc.py:283-364), bf16 only: the
 *   projection launch forms x_new[t, r, :] = sum_s h_res_prev[t, r, s]
 *   x_old[t, s, :] + h_post_prev[t, r] out[t, :] from x_old and out as it
 *   loads them, writes it (row stride ld_new) and feeds it to the matrix
 *   cores, so the separate update pass (read x_old, write x_new) and the
 *   projection's read of x_new become one pass; the per-token launch then
 *   reads x_new as walsh_mhc_pre_wide_fwd reads x.  x_new is bitwise what
 *   walsh_mhc_post_fwd writes; h_pre / h_post / h_res / layer_in equal
 *   walsh_mhc_pre_wide_fwd's on x_new up to the float32 summation order of
 *   the projection.  C a multiple of 32 up to 4096, row strides multiples of
 *   8, 16-byte aligned buffers; workspace as walsh_mhc_pre_wide_workspace;
 *   x_new may not alias x_old, nor the new h_post / h_res the previous
 *   ones. */
int walsh_mhc_post_pre_wide_fwd(const void *x_old, int64_t ld_old, const void *out, int64_t ld_out,
                                const float *h_res_prev, const float *h_post_prev, void *x_new, int64_t ld_new,
                                int64_t M, int64_t n, int64_t C, const void *phi_frag32, const float *coef,
                                const float *bias, float rms_eps, int64_t n_iter, float sk_eps, float *h_pre,
                                float *h_post, float *h_res, void *layer_in, int64_t ld_in, const float *norm_w,
                                float norm_eps, void *workspace, int64_t workspace_bytes, int dtype, void *stream);

/* walsh_mhc_post_fwd: x_new = H_res @ x + H_post^T (x) out
 *   (src/model/mhc.py:366-381).  out [M, C] row stride ld_out; x_new may not
 *   alias x. */
int walsh_mhc_post_fwd(const void *x, int64_t ldx, const void *out, int64_t ld_out, const float *h_res,
                       const float *h_post, void *x_new, int64_t ld_new, int64_t M, int64_t n, int64_t C, int dtype,
                       void *stream);

/* Training (the autograd torch derives for mHCResidualStream.forward,
 * src/model/mhc.py:366-381); dense rows: x, dx, d_new [M][n][C];
 * layer_in, d_layer_in, out, d_out [M][C] (all of dtype); h_pre, h_post
 * [M][n], h_res [M][n][n] and their gradients float32; n <= 4, C % 4 == 0.
 * walsh_mhc_aggregate_fwd: layer_in = H_pre @ x (mhc.py:366), float32 sums.
 * walsh_mhc_aggregate_bwd: dx = H_pre^T d_layer_in, dh_pre[s] = <d_layer_in, x_s>.
 * walsh_mhc_post_bwd: for x_new = H_res @ x + H_post^T (x) out:
 *   dx_s = sum_i H_res[i][s] d_new_i, d_out = sum_i H_post[i] d_new_i,
 *   dh_res[i][s] = <d_new_i, x_s>, dh_post[i] = <d_new_i, out>.
 *   One wavefront per token; sums over C in a fixed order. */
int walsh_mhc_aggregate_fwd(const void *x, const float *h_pre, void *layer_in, int64_t M, int64_t n, int64_t C,
                            int dtype, void *stream);
int walsh_mhc_aggregate_bwd(const void *x, const float *h_pre, const void *d_layer_in, void *dx, float *dh_pre,
                            int64_t M, int64_t n, int64_t C, int dtype, void *stream);
int walsh_mhc_post_bwd(const void *x, const void *out, const float *h_res, const float *h_post, const void *d_new,
                       void *dx, void *d_out, float *dh_res, float *dh_post, int64_t M, int64_t n, int64_t C,
                       int dtype, void *stream);

/* ------------------------------------------------------------------ A10-A13
 * Hadamard mixture-of-experts FFN (src/model/moe.py:306-560).  Expert e owns
 * the 32-wide feature block x[:, 32e:32e+32]; E <= 128 experts; each token
 * is routed to k = min(max_experts, E) <= 8 experts.
 *
 * Routing outputs (shared by walsh_moe_route_fwd and walsh_moe_topk_fwd):
 *   topk_idx [M, k] int32, experts by decreasing probability (equal
 *     probabilities: lower expert index first);
 *   topk_w [M, k] float32, probs / max(sum of the selected probs, 1e-8);
 *   count [n_part][E] int32 and probsum [n_part][E] float32: per-workgroup
 *     partial sums of the tokens routed to each expert and of the softmax
 *     probabilities (for the balance loss); the totals are the sums over
 *     the first index (walsh_moe_scatter forms them).  Rows a call does not
 *     use are zeroed; 1 <= n_part <= 65536.  Partial sums replace
 *     same-address global atomics, which serialise across the chip;
 *   probs / mask / weights_dense [M, E] float32 are optional (NULL skips):
 *     the three outputs of HadamardRouter.forward.
 *
 * walsh_moe_route_fwd: HadamardRouter.forward (src/model/moe.py:418-447),
 *   logits = W2 silu(W1 x) (no biases), softmax (float32), top-k,
 *   renormalised weights.  x [M, C] (row stride ldx, dtype), W1 [H1, C] and
 *   W2 [E, H1] given in matrix-core fragment order (dtype elements):
 *   w1_frag[H1/16][C/16][64][4] holds W1[16a + l%16][16b + 4(l/16) + j] and
 *   w2_frag[ceil(E/16)][H1/16][64][4] holds W2[16a + l%16][16b + 4(l/16) + j]
 *   (rows >= E zero).  With dtype WALSH_BF16 the hidden activations and the
 *   logits are rounded to bfloat16 where torch.autocast rounds them.  If y
 *   is not NULL, the output blocks y[t, 32e:32e+32] (ydtype, row stride ldy)
 *   of every unselected expert are set to zero.  Needs C % 16 == 0,
 *   H1 % 16 == 0, E <= 64.
 */
int walsh_moe_route_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H1, const void *w1_frag,
                        const void *w2_frag, int64_t E, int64_t k, float *probs, float *mask, float *weights_dense,
                        int *topk_idx, float *topk_w, int *count, float *probsum, int64_t n_part, void *y,
                        int64_t ldy, int dtype, int ydtype, void *stream);

/* walsh_moe_router_wide_fwd: HadamardRouter.forward (src/model/moe.py:
 *   418-447) for wide models (n_embd 4096: W1 4096 -> 1024, W2 -> 128
 *   experts), bf16 only, on matrix cores: h = silu(x W1^T) [M, H], then
 *   logits = h W2^T with the softmax / top-k / routing outputs of
 *   walsh_moe_route_fwd.  W1 [H, C] and W2 [E, H] are plain row-major bf16
 *   matrices (the Linear weights cast to bf16).  The first product, SiLU's
 *   result and the logits are rounded to bfloat16 where torch.autocast
 *   rounds them.  work: walsh_moe_router_wide_workspace_bytes(M, H, E)
 *   bytes, 256-byte aligned; its first M*H bf16 values hold h afterwards.
 *   Needs C % 256 == 0, H % 128 == 0, H <= 1024, E % 4 == 0, 16-byte
 *   aligned operands and rows. */
int64_t walsh_moe_router_wide_workspace_bytes(int64_t M, int64_t H, int64_t E);
int walsh_moe_router_wide_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H, const void *w1,
                              const void *w2, int64_t E, int64_t k, void *work, int64_t work_bytes, float *probs,
                              float *mask, float *weights_dense, int *topk_idx, float *topk_w, int *count,
                              float *probsum, int64_t n_part, void *y, int64_t ldy, int ydtype, void *stream);

/* walsh_moe_decode_fwd: the whole HadamardMoE.forward (src/model/moe.py:
 *   512-542: HadamardRouter.forward :418-447, then FastMoEExperts.forward
 *   :337-380 on the routed pairs) for 1..4 tokens (decode) of a wide bf16
 *   model, in one launch: the router as walsh_moe_router_wide_fwd (C ==
 *   32 E, C % 256 == 0, hidden H % 128 == 0 and <= 1024, E % 4 == 0), the
 *   experts as walsh_moe_experts_fwd (expert hidden He in {64, 128, 256},
 *   fragments from the same layout) with y [M, >= 32E] (ydtype) written
 *   whole: expert output * routing weight in the routed blocks, zeros in
 *   the others.  Outputs equal the router / scatter / experts calls bitwise;
 *   partial row t of count / probsum holds token t's counts and
 *   probabilities (rows M.. of n_part zero), as the per-token rows of
 *   walsh_moe_router_wide_fwd.  work: walsh_moe_decode_workspace_bytes(M, H, E) bytes,
 *   256-byte aligned.  sync: one unsigned counter, zero before the first
 *   call; each call leaves it at zero.  Calls that share a counter must not
 *   overlap. */
int64_t walsh_moe_decode_workspace_bytes(int64_t M, int64_t H, int64_t E);
int walsh_moe_decode_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H, const void *w1, const void *w2,
                         int64_t E, int64_t k, int64_t He, const uint8_t *gate_frag, const uint8_t *up_frag,
                         const uint8_t *down_frag, const float *gammas, void *work, int64_t work_bytes, unsigned *sync,
                         float *probs, float *mask, float *weights_dense, int *topk_idx, float *topk_w, int *count,
                         float *probsum, int64_t n_part, void *y, int64_t ldy, int ydtype, void *stream);

/* walsh_moe_experts_bwd: backward of FastMoEExperts.forward (src/model/moe.py
 *   :337-380, autograd of its einsums, SiLU and routing product, with the
 *   MoE STE of :289-294) over the routed pairs of a walsh_moe_scatter
 *   grouping (list, offset), float32: x, dout [M, >= 32E] (row strides ldx,
 *   ldd), the packed codes (gate / up [E][H][8], down [E][32][H/4]), gammas
 *   [3] and topk_w [M*k].  Writes dx[t, 32e:32e+32] of every routed pair
 *   (other blocks untouched: zero them first), d_pair_w [M*k] (gradient of
 *   each pair's routing weight) and clamp(dW, -2, 2) of the three weight
 *   tensors (gate / up [E][H][32], down [E][32][H]; NULL skips).  Hidden H
 *   <= 128, multiple of 16.  work: walsh_moe_experts_bwd_workspace_bytes(E,
 *   H) bytes. */
int64_t walsh_moe_experts_bwd_workspace_bytes(int64_t E, int64_t H);
int walsh_moe_experts_bwd(const float *x, int64_t ldx, const float *dout, int64_t ldd, int64_t M, int64_t E,
                          int64_t k, int64_t H, const uint8_t *gate_packed, const uint8_t *up_packed,
                          const uint8_t *down_packed, const float *gammas, const int *list, const int *offset,
                          const float *topk_w, float *dx, int64_t ldgx, float *d_pair_w, float *dgate, float *dup,
                          float *ddown, void *work, int64_t work_bytes, void *stream);

/* walsh_moe_topk_fwd: the softmax / top-k / renormalisation part of
 *   HadamardRouter.forward (src/model/moe.py:432-445) from given float32
 *   logits [M, E] (contiguous). */
int walsh_moe_topk_fwd(const float *logits, int64_t M, int64_t E, int64_t k, float *probs, float *mask,
                       float *weights_dense, int *topk_idx, float *topk_w, int *count, float *probsum,
                       int64_t n_part, void *stream);

/* walsh_moe_scatter: per-expert lists of the M*k (token, slot) pairs, the
 *   grouping that replaces the dense all-expert einsum of
 *   FastMoEExperts.forward (src/model/moe.py:363-374).  From the partial
 *   sums of a routing call it forms count [E] and probsum [E] (totals),
 *   offset [E+1] = exclusive scan of count and tile_off [E+1] = exclusive
 *   scan of ceil(count/16); list [M*k] then holds the pair ids t*k + j
 *   grouped by expert (order inside a group unspecified).  cursor [E] is
 *   scratch. */
int walsh_moe_scatter(const int *topk_idx, int64_t M, int64_t E, int64_t k, const int *count_part,
                      const float *probsum_part, int64_t n_part, int *count, float *probsum, int *cursor, int *list,
                      int *offset, int *tile_off, void *stream);

/* walsh_moe_experts_fwd: FastMoEExperts.forward (src/model/moe.py:337-380)
 *   on the routed pairs only: y[t, 32e:32e+32] = w * down_e(silu(gate_e x_e)
 *   * up_e x_e) for x_e = x[t, 32e:32e+32], with ternary weights
 *   code * gamma (moe.py:268-303).  Expert hidden size H in {64, 128, 256}.
 *   Packed codes (2-bit, pack_ternary_weights byte order) in fragment order:
 *   gate_frag/up_frag [E][H/16][2][64]: byte of row 16a + l%16, K bytes
 *   4c + l/16 (c = second index); down_frag [E][2][H/16][64]: byte of row
 *   16m + l%16, K byte 4b + l/16.  gammas [3] float32 (gate, up, down).
 *   Writes only the selected blocks of y (the router zero-fills the rest).
 *   (dtype, ydtype) is (f32, f32), (bf16, bf16) or (bf16, f32); bf16
 *   rounds where torch.autocast rounds. */
int walsh_moe_experts_fwd(const void *x, int64_t ldx, void *y, int64_t ldy, int64_t M, int64_t E, int64_t k,
                          int64_t H, const uint8_t *gate_frag, const uint8_t *up_frag, const uint8_t *down_frag,
                          const float *gammas, const int *list, const int *offset, const int *tile_off,
                          const int *count, const float *topk_w, int dtype, int ydtype, void *stream);

/* walsh_moe_ffn_fwd: the whole HadamardMoE.forward (src/model/moe.py:512-542)
 *   in one launch for n_embd 512 (E = 16 experts, router 512 -> 128 -> 16),
 *   bf16 input: router, routing (outputs as walsh_moe_route_fwd, zeroed
 *   blocks of unselected experts included) and the routed experts.
 *   Fragment orders (bf16 elements for the router, 16-bit code pairs for the
 *   experts; l = lane 0..63, s = slot):
 *     w1_frag [8][16][64][8]: W1[16a + l%16][32b + 8(l/16) + s];
 *     w2_frag [8][64][4]: W2[l%16][16c + 4(l/16) + s] (rows >= E zero);
 *     gate_frag / up_frag [16][64][H/16]: packed bytes 2(l/16) (low) and
 *       2(l/16) + 1 (high) of row 16a + l%16 (rows of 8 bytes);
 *     down_frag [16][64][2][H/32]: packed bytes 8c + l/16 (low) and
 *       8c + 4 + l/16 (high) of row 16m + l%16 (rows of H/4 bytes).
 *   count [n_part][E] and probsum [n_part][E]: partial sums as above.
 *   H in {64, 128}, k <= 8, ydtype WALSH_F32 or WALSH_BF16. */
int walsh_moe_ffn_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, const void *w1_frag, const void *w2_frag,
                      int64_t E, int64_t k, int64_t H, const uint16_t *gate_frag, const uint16_t *up_frag,
                      const uint16_t *down_frag, const float *gammas, int *topk_idx, float *topk_w, int *count,
                      float *probsum, int64_t n_part, void *y, int64_t ldy, int dtype, int ydtype, void *stream);

/* ------------------------------------------------------------------ channel modulation
 * HadamardChannelModulation (src/model/moe.py:610-771).  Rows come in G
 * groups of T rows (the module's [B, T, C] input, G = B; mHCLlamaBlock
 * passes the [B*n, T, C] view of its streams, src/model/mhc.py:528-532):
 * row (g, t) at x + (g*T + t)*ldx.  C % 4 == 0, C <= 4096; n_blocks divides
 * C (block b = columns [b*C/n_blocks, (b+1)*C/n_blocks)).  bf16 rows 8-byte
 * aligned, float32 rows 16-byte aligned, strides multiples of 4.
 *
 * walsh_chanmod_workspace_bytes: float scratch for the per-chunk column
 *   sums of walsh_chanmod_fwd / walsh_chanmod_bwd.
 * walsh_chanmod_fwd: the module's forward with the scale / shift MLP
 *   (moe.py:676-727, ternary branch :753-762), for xn = x, or, if norm_w
 *   (float32 [C], 16-byte aligned) is non-NULL, xn = x * rsqrt(mean(x^2) +
 *   eps) * norm_w (the RMSNorm in front of it, chassis.py:96-106):
 *     bulk[g] = mean_t xn[g, t];  h = silu(w1 bulk[g]);  m = w2 h
 *     scale[g][b] = 1 + clamp(*scale_temp, 0.1, 0.5) * tanh(m[b]);
 *     shift[g][b] = m[n_blocks + b]
 *     y = (add_input ? x : 0) + xn + residual_scale * (xn*scale + shift_scale*shift - xn)
 *   w1 float32 [hidden][C], w2 float32 [2*n_blocks][hidden] (the context
 *   MLP's weights: code * gamma for the ternary module, walsh_ternary_quantize's
 *   `scaled`, or the latent weights for use_ternary=False); scale_temp a
 *   device float.  scale_shift float32 [G][2*n_blocks] receives scale then
 *   shift of each group (the module's statistics come from it).  y may not
 *   alias x.  Everything is computed in float32; y is rounded to dtype once.
 * walsh_chanmod_apply: the per-block modulation alone, ChannelModFunction's
 *   forward (moe.py:116-153, :202-233): y = x + residual_scale * (x*scale +
 *   shift_scale*shift - x) with scale / shift float32, element (g, b) at
 *   g*ld_ss + b.
 * walsh_chanmod_bwd: ChannelModFunction's backward (moe.py:155-199,
 *   :235-256) for the output gradient gy:
 *     gx = gy * (1 + residual_scale * (scale - 1))
 *     dscale[g][b] = residual_scale * sum over the group's rows and block b of gy*x
 *     dshift[g][b] = shift_scale * residual_scale * sum of gy
 *   gy, x and gx share dtype; the sums are float32 in a fixed order
 *   (deterministic). */
int64_t walsh_chanmod_workspace_bytes(int64_t G, int64_t T, int64_t C);
int walsh_chanmod_fwd(const void *x, int64_t ldx, int64_t G, int64_t T, int64_t C, const float *norm_w, float eps,
                      const float *w1, int64_t hidden, const float *w2, int64_t n_blocks, const float *scale_temp,
                      float residual_scale, float shift_scale, int add_input, void *y, int64_t ldy,
                      float *scale_shift, int dtype, void *workspace, int64_t workspace_bytes, void *stream);
int walsh_chanmod_apply(const void *x, int64_t ldx, int64_t G, int64_t T, int64_t C, int64_t n_blocks,
                        const float *scale, const float *shift, int64_t ld_ss, float residual_scale,
                        float shift_scale, void *y, int64_t ldy, int dtype, void *stream);
int walsh_chanmod_bwd(const void *gy, int64_t ldg, const void *x, int64_t ldx, int64_t G, int64_t T, int64_t C,
                      int64_t n_blocks, const float *scale, int64_t ld_ss, float residual_scale, float shift_scale,
                      void *gx, int64_t ldgx, float *dscale, float *dshift, int dtype, void *workspace,
                      int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* WALSH_H */
