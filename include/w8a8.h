/*
 * w8a8.h - C ABI of the MI355X (gfx950) W8A8 INT8 linear path.
 *
 * Plain C: fixed-width integers, raw device pointers, an opaque stream
 * handle (a hipStream_t passed as void*). No torch types. Every entry point
 * takes a pointer to an argument struct whose first field is the struct size
 * (checked against sizeof, like the reference's AttentionArgs static_assert,
 * patches/kitchen_attention_native/attention.cu:5-18,79), validates shapes,
 * strides and alignment before launching, enqueues work on the caller's
 * stream without synchronising, and returns a w8a8_status code
 * (the reference's native entry returns a cudaError_t, attention.cu:79-101).
 *
 * The caller owns and allocates every input, output and workspace buffer;
 * the library allocates no device memory and keeps no state beyond a
 * per-thread error message. Calls on different streams may run concurrently.
 *
 * Numerics (all float ops are IEEE binary32 round-to-nearest-even, no FMA
 * contraction):
 *   quantize:  s = max(amax * fp32(1/127), fp32(1e-30)),
 *              q = clamp(rne(x / s), -128, 127)         (IEEE division)
 *   ConvRot256: per 256-column group, four radix-4 stages (strides 1,4,16,64)
 *              of the regular H4 butterfly ((p+q)+r)+s, then * fp32(1/16)
 *   GEMM:      C[m][n] = sum_k A[m][k] * B[n][k]  (int32, exact)
 *   ROW epilogue:    y = (f32(C) * a[m]) * w[n]   [+ f32(bias[n])]
 *   COLUMN epilogue: y = f32(C) * (a[m] * w[n])   [+ f32(bias[n])]
 *   residual:  out = f16(f32(res[m][n]) + f32(f16(y)))
 *   gated residual: out = f16(fma(f32(f16(y)), gate[label[m]][n], f32(res[m][n])))
 *              (one rounding, as __fmaf_rn)
 */
#ifndef W8A8_H
#define W8A8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W8A8_ABI_VERSION 13

typedef enum w8a8_status {
  W8A8_OK = 0,
  W8A8_ERR_INVALID = 1,     /* bad pointer, shape, stride, alignment or size */
  W8A8_ERR_UNSUPPORTED = 2, /* valid request outside what the kernels cover */
  W8A8_ERR_LAUNCH = 3       /* the HIP runtime refused a launch */
} w8a8_status;

typedef enum w8a8_dtype {
  W8A8_F16 = 1,
  W8A8_BF16 = 2,
  W8A8_F32 = 3,
  W8A8_I32 = 4,
  W8A8_I8 = 5
} w8a8_dtype;

typedef enum w8a8_epilogue {
  W8A8_EPI_INT32 = 0,  /* raw int32 accumulators */
  W8A8_EPI_ROW = 1,    /* (C * a) * w, parallel_int8.dequantize order */
  W8A8_EPI_COLUMN = 2  /* C * (a * w), column epilogue order */
} w8a8_epilogue;

/*
 * Dynamic per-row absmax quantization, optionally after ConvRot256.
 * Replaces: patches/parallel_int8.py:26-43 (quantize),
 *           patches/dit_column_linear.py:13-21 (_prepare_activation),
 *           patches/tilelang_row_quant.py:26-46,81-86 (quantizer with an
 *           external row maximum).
 * x: [rows, cols] of x_dtype (F16, BF16, F32), row stride ldx elements.
 * convrot: 0 (none) or 256 (ConvRot256 before the absmax).
 * round_rotated: with convrot, 1 rounds the rotated values to x_dtype before
 *   the absmax (the column path's rotation returns a tensor of x's dtype,
 *   patches/dit_column_linear.py:18-19); 0 keeps them in FP32 (the fused
 *   rotate-and-quantize route of patches/parallel_int8.py:32-36).
 * row_max: optional [rows] external absmax (e.g. a global maximum over
 *   tensor-parallel owners); NULL computes the row's own absmax.
 * q: [rows, cols] int8, row stride ldq. scale: [rows] fp32.
 * row_max_out: optional [rows] fp32, receives the row's own absmax of the
 *   (rotated) values: the local maximum a tensor-parallel owner contributes
 *   to the MAX exchange (patches/tilelang_row_quant.py:49-62 maximum_kernel,
 *   :136-146). Requires row_max == NULL. With q == scale == NULL only the
 *   maximum is computed (the maximum phase).
 * convrot_signs: optional [cols] sign words for a seeded ConvRot (with
 *   convrot, 16-byte aligned): 0 keeps column j, 0x80000000 negates it
 *   before the rotation, which becomes diag(s) then H (s = +-1; weights
 *   rotated the same way keep the GEMM unchanged). NULL: s = +1, the
 *   reference's ConvRot. No counterpart in the reference (an option of the
 *   configuration it is benchmarked on).
 * Requirements: cols % 16 == 0 (cols % 256 == 0 with convrot), x, q 16-byte
 *   aligned, ldx * elem and ldq multiples of 16 bytes.
 */
typedef struct W8A8QuantArgs {
  uint32_t struct_size;
  int32_t x_dtype;
  const void* x;
  int64_t ldx;
  int64_t rows;
  int64_t cols;
  int32_t convrot;
  int32_t round_rotated;
  const float* row_max;
  int8_t* q;
  int64_t ldq;
  float* scale;
  void* stream;
  float* row_max_out;
  const uint32_t* convrot_signs;
} W8A8QuantArgs;

int w8a8_quantize_rows(const W8A8QuantArgs* args);

/*
 * FC2 prologue: FP32 SwiGLU -> ConvRot256 -> row absmax -> quantize, fused,
 * with no FP32 round trip through memory.
 * Replaces: patches/tilelang_swiglu_quant.py:11-64 (fused_kernel, phases
 *           stored / maximum / recompute), :67-92 (prepare, fused_stored),
 *           patches/tilelang_row_quant.py:26-46 (external-max quantizer).
 * x: [rows, 2*width] of x_dtype (F16 or F32): gate in columns [0, width),
 *   up in [width, 2*width); row stride ldx elements. width % 256 == 0.
 * Per element: a = (g / (1 + exp(-g))) * u in FP32 (exp is this library's
 *   own correctly-rounded-to-about-1-ulp Cody-Waite/Cephes evaluation).
 * row_max: optional [rows] external (global) absmax of the rotated values.
 * row_max_out: optional [rows] output of the local absmax.
 * group_max: optional [rows, width/256] output of per-group absmax.
 * q: [rows, width] int8 (row stride ldq) or NULL (maximum phase only).
 * scale: [rows] fp32 (required when q is non-NULL).
 * convrot_signs: optional [width] sign words applied to the SwiGLU output
 *   before its rotation, as in w8a8_quantize_rows.
 */
typedef struct W8A8SwigluArgs {
  uint32_t struct_size;
  int32_t x_dtype;
  const void* x;
  int64_t ldx;
  int64_t rows;
  int64_t width;
  const float* row_max;
  float* row_max_out;
  float* group_max;
  int8_t* q;
  int64_t ldq;
  float* scale;
  void* stream;
  const uint32_t* convrot_signs;
} W8A8SwigluArgs;

int w8a8_swiglu_quantize(const W8A8SwigluArgs* args);

/*
 * DiT modulated RMSNorm, optionally fused with ConvRot256 and the per-row
 * quantizer (the QKV / FC1 input preparation), so the normalized tensor
 * need not make an HBM round trip before its quantization.
 * Replaces: patches/tilelang_dit_fusion.py:10-36 (norm_kernel) and
 *           :127-135 (modulated_norm), patches/h3_tensor_flow.py:134-142
 *           (modulated_norm), then patches/dit_column_linear.py:13-21
 *           (_prepare_activation) on its output.
 * x: [rows, cols] F16 or BF16, row stride ldx elements.
 * weight: optional [cols] fp32 norm gain (NULL: no gain).
 * mod_shift, mod_scale: optional fp32 AdaLN tables [mod_rows, ld_mod] (both
 *   or neither); labels: int32 [rows], each row's table row in
 *   [0, mod_rows) (values outside are clamped into that range).
 * Per row, in fp32 (round to nearest even, no contraction):
 *   ss   = sum of x*x in a fixed order: lane l of 64 adds, in order, the
 *          squares of elements 16u..16u+15 of units u = l, l+64, l+128, ...;
 *          the 64 partials then meet in an xor butterfly (offsets 32..1)
 *   inv  = 1 / sqrt(ss * fp32(1/cols) + eps)      (IEEE sqrt and division)
 *   y    = x_dtype(((((x * inv) * w) * (1 + mod_scale[l])) + mod_shift[l]))
 * y: optional [rows, cols] x_dtype output of the normalized rows (ldy).
 * convrot, round_rotated, q, ldq, q_scale, convrot_signs: as
 *   w8a8_quantize_rows applied to y. q NULL runs the norm alone (y
 *   required).
 * Requirements: cols % 16 == 0 (cols % 256 == 0 with convrot and q), x, y,
 *   q and every table 16-byte aligned with 16-byte row strides.
 */
typedef struct W8A8NormArgs {
  uint32_t struct_size;
  int32_t x_dtype;
  const void* x;
  int64_t ldx;
  int64_t rows;
  int64_t cols;
  const float* weight;
  const float* mod_shift;
  const float* mod_scale;
  int64_t ld_mod;
  int32_t mod_rows;
  float eps;
  const int32_t* labels;
  void* y;
  int64_t ldy;
  int32_t convrot;
  int32_t round_rotated;
  int8_t* q;
  int64_t ldq;
  float* q_scale;
  void* stream;
  const uint32_t* convrot_signs;
} W8A8NormArgs;

int w8a8_norm_quantize(const W8A8NormArgs* args);

/*
 * Per-head RMS normalization with FP32 statistics and gains, then split-half
 * RoPE, of the Q and K parts of a packed QKV projection output.
 * Replaces: patches/tilelang_fp32_rms_rope.py:6-66 (kernel, execute) and the
 *           Kitchen rms_rope_split_half call of patches/tp_dit.py:296-309.
 * packed: [rows, >= 2*heads*dim] of in_dtype (F16 or F32), row stride ldp;
 *   Q heads in columns [0, heads*dim), K heads in [heads*dim, 2*heads*dim).
 * freqs: [rows, rot_dim/2, 2, 2] of freq_dtype (F16 or F32), contiguous: for
 *   pair p the 2x2 matrix F applied to (x[p], x[p + rot_dim/2]).
 * q_gain, k_gain: [dim] fp32.
 * Per head vector x (dim = 128), in fp32 (round to nearest even):
 *   ss  = sum of x*x in a fixed order: the vector is 16 slices of 8 elements;
 *         slice i adds its squares in order, then the 16 partials meet in an
 *         xor butterfly (offsets 8, 4, 2, 1)
 *   inv = 1 / sqrt(ss * fp32(1/dim) + eps)           (IEEE sqrt and division)
 *   n   = (x * inv) * gain
 *   d < rot_dim: out = fma(n[partner], F[p][s][1-s], n[d] * F[p][s][s]) with
 *         p = d mod rot_dim/2, s = d div rot_dim/2, partner = the other half
 *   d >= rot_dim: out = n[d]
 * q_out, k_out: [rows, heads, dim] of out_dtype (F16 or F32), contiguous.
 * Requirements: dim == 128, rot_dim even with 0 < rot_dim <= 128; packed,
 *   freqs, gains and outputs 16-byte aligned, ldp * elem a multiple of 16.
 */
typedef struct W8A8RmsRopeArgs {
  uint32_t struct_size;
  int32_t in_dtype;
  const void* packed;
  int64_t ldp;
  int64_t rows;
  int32_t heads;
  int32_t dim;
  int32_t rot_dim;
  int32_t freq_dtype;
  const void* freqs;
  const float* q_gain;
  const float* k_gain;
  float eps;
  int32_t out_dtype;
  void* q_out;
  void* k_out;
  void* stream;
} W8A8RmsRopeArgs;

int w8a8_rms_rope(const W8A8RmsRopeArgs* args);

/*
 * INT8 attention for 128-wide heads, in two calls like the reference's
 * prepared Kitchen route (patches/h3_operator_policy.py:173-209:
 * ck.prequantize_int8_attention, then ck.int8_attention_from_prequantized;
 * patches/kitchen_attention.py:227-238 int8_attention; the native launcher
 * patches/kitchen_attention_native/attention.cu:20-66 h3_attention). The
 * numerics are those of the reference's vendored kernel
 * (kitchen_attention_native/vendor/qk_int_sv_i8_cuda.cuh, attn_utils.cuh) for
 * key blocks of CTA_K = 128, with the SageAttention quantizer assumed for
 * Kitchen's absent one:
 *   prepare: codes sat(round half away(x / s)) with s = amax / 127 + 1e-7; q rows
 *     32 G + 8 i + j share the scale of (G, j); k is centred per channel
 *     (its fp32 mean) and key 8 t + 2 c + e of a 128-key block shares the
 *     scale of (block, c); v takes one scale per channel. v is written
 *     transposed: vt8[c][128 j + 32 u + p] holds key 128 j + 32 u + 8 g + 4 h
 *     + i of channel c for p = 16 h + 4 g + i; vsum[j][c] = 128 * the sum of
 *     block j's v codes of channel c.
 *   attention: one online pass over the 128-key blocks in the exp2 domain:
 *     the block's maximum per K-scale group, tile_m = max over the groups of
 *     fma(mt, fp32(c0 * fp32(qs * ks)), -S_U8_OFFSET) (c0 = sm_scale *
 *     log2(e)), u8 probabilities sat(rne(exp2(fma(S, ts, -tile_m)))) relative
 *     to the block's own maximum, FP32 rescaling of the running output and of
 *     the four group denominators, P.V exact in int32 and added with one FMA
 *     of the block scale; output (O * (1 / sum of denominators)) * vs[c]
 *     (hardware exp2; nk <= 131072).
 * q, k, v: [b, h, nq|nk, d] with element strides {batch, head, token} given
 * per tensor and the d == 128 channels contiguous (e.g. the q, k and v
 * columns of a packed [tokens, 3 * h * d] QKV projection, or contiguous
 * [b, h, n, d] tensors); the output takes strides the same way. Every stride
 * and base address must be a multiple of 16 bytes.
 */
typedef struct W8A8AttnPrepareArgs {
  uint32_t struct_size;
  int32_t in_dtype;        /* W8A8_F16 or W8A8_F32 */
  const void* q;
  const void* k;
  const void* v;
  int64_t b;
  int64_t h;
  int64_t nq;
  int64_t nk;
  int32_t d;
  float sm_scale;          /* > 0 (checked; the attention call takes its own) */
  int64_t q_strides[3];    /* element strides of q's batch, head and token dims */
  int64_t k_strides[3];
  int64_t v_strides[3];
  int8_t* q8;              /* [b, h, nq, d] */
  float* qs;               /* [b, h, nq]: each row's group scale */
  int8_t* k8;              /* [b, h, nkp, d], nkp = 128 * ceil(nk / 128) */
  float* ks;               /* [b, h, nkp / 128, 4]: the four group scales of each block */
  int8_t* vt8;             /* [b, h, d, nkp] */
  float* vs;               /* [b, h, d] */
  int32_t* vsum;           /* [b, h, nkp / 128, d]: 128 * each block's sum of v codes */
  void* workspace;         /* w8a8_attention_workspace_size(b, h, nk) bytes */
  int64_t workspace_bytes;
  void* stream;
} W8A8AttnPrepareArgs;

int w8a8_attention_prepare(const W8A8AttnPrepareArgs* args);

/* Scratch bytes w8a8_attention_prepare needs (key statistics, V divisors). */
int64_t w8a8_attention_workspace_size(int64_t b, int64_t h, int64_t nk);

typedef struct W8A8AttentionArgs {
  uint32_t struct_size;
  int32_t out_dtype;       /* W8A8_F16 or W8A8_F32 */
  const int8_t* q8;
  const float* qs;
  const int8_t* k8;
  const float* ks;
  const int8_t* vt8;
  const float* vs;
  const int32_t* vsum;
  int64_t b;
  int64_t h;
  int64_t nq;
  int64_t nk;
  int32_t d;
  float sm_scale;          /* > 0; the reference's default is 1/sqrt(d) */
  void* out;               /* [b, h, nq, d] of out_dtype, element strides out_strides */
  int64_t out_strides[3];  /* batch, head, token */
  void* stream;
} W8A8AttentionArgs;

int w8a8_attention(const W8A8AttentionArgs* args);

/*
 * INT8 GEMM on gfx950 i8 MFMA with a fused epilogue.
 * Replaces: patches/parallel_int8.py:46-50 (int_mm),
 *           patches/optimized_tp.py:34-43 (native_int_mm),
 *           patches/dit_column_linear.py:51-57 (_column_accumulate)
 *   fused with patches/parallel_int8.py:53-69 (dequantize, ROW order),
 *   patches/tilelang_column_epilogue.py:10-40 (COLUMN order) and
 *   patches/h3_tensor_flow.py:130-131 (residual_add).
 * a: [m, k] int8 activations (row stride lda); b: [n, k] int8 weights
 *   (row stride ldb) - both K-contiguous ("TN").
 * row_scale: [m] fp32; col_scale: [n] fp32 with col_scale_stride 1, or a
 *   scalar with stride 0. Unused for W8A8_EPI_INT32.
 * bias: optional [n] of bias_dtype (F16 or F32), added after the products.
 * residual: optional [m, n] F16 (row stride ldr); requires out_dtype F16.
 *   May alias out (in-place residual update).
 * gate, gate_labels, ldg: optional DiT modulation gate (requires residual):
 *   gate fp32 table [R, ldg] (ldg >= n), gate_labels int32 [m] (each row's
 *   table row, in [0, R)); the residual update becomes
 *   f16(fma(f32(f16(y)), gate[gate_labels[m]][n], f32(res))).
 *   Replaces patches/tilelang_dit_fusion.py:56-77 (row_gate_kernel) and
 *   patches/h3_tensor_flow.py:145-152 (gated_add).
 * out: [m, n] of out_dtype (I32 for EPI_INT32; F16, BF16 or F32 otherwise),
 *   row stride ldc.
 * workspace: optional device buffer of workspace_bytes bytes (16-byte
 *   aligned, any contents). When w8a8_gemm_workspace_size() is non-zero for
 *   the shape and the workspace holds at least that many bytes, grids too
 *   small to fill the GPU split K across workgroups: each writes exact int32
 *   partial sums into the workspace and a second kernel adds them and runs
 *   the epilogue (the result is bit-identical to the unsplit GEMM). NULL / 0
 *   never splits. Calls that share a workspace must not overlap; calls in
 *   sequence may share one, and a captured graph may replay it.
 * rope: optional RMS-RoPE epilogue (W8A8RopeEpilogue) for a packed QKV
 *   projection: the Q and K heads of the output are normalized and rotated
 *   as w8a8_rms_rope would on the stored fp16 output, in the same kernel, so
 *   the QKV output makes no second HBM trip (replaces
 *   patches/tilelang_fp32_rms_rope.py:6-66 after the QKV projection,
 *   patches/tp_dit.py:288-301). Requires out_dtype F16, no bias, residual
 *   or gate, (rot_dim / 2) % 8 == 0, m > 64, k % 128 == 0, 16-byte aligned
 *   output rows, operands spanning < 4 GB; never splits K. Other requests return
 *   W8A8_ERR_UNSUPPORTED (use w8a8_rms_rope on the output instead).
 * Requirements: k % 16 == 0; a, b 16-byte aligned; lda, ldb % 16 == 0;
 *   out element-aligned (rows are written with vector stores when out is
 *   16-byte aligned and ldc % 4 == 0).
 */
/* The RMS-RoPE epilogue of w8a8_gemm (see W8A8GemmArgs.rope). Output
 * columns [0, heads*128) are the Q heads and [heads*128, 2*heads*128) the K
 * heads (the numerics of w8a8_rms_rope with dim 128); later columns (V) are
 * stored unchanged. freqs of freq_dtype (F16 or F32), in freq_layout
 *   W8A8_ROPE_MATRICES: [m, rot_dim/2, 2, 2], F[p][s][t] (the reference's);
 *   W8A8_ROPE_PAIRS: [m, 2, rot_dim/2, 2], entry [s][p] = (F[p][s][s],
 *     F[p][s][1-s]) - the same values ordered so a lane's eight rotations
 *     are one contiguous run (built once per forward, see the package's
 *     rms_rope.pack_freqs);
 * q_gain, k_gain: [128] fp32; all 16-byte aligned. */
enum { W8A8_ROPE_MATRICES = 0, W8A8_ROPE_PAIRS = 1 };
typedef struct W8A8RopeEpilogue {
  int32_t heads;
  int32_t rot_dim;
  int32_t freq_dtype;
  float eps;
  int32_t freq_layout;     /* W8A8_ROPE_MATRICES or W8A8_ROPE_PAIRS */
  int32_t reserved;
  const void* freqs;
  const float* q_gain;
  const float* k_gain;
} W8A8RopeEpilogue;

typedef struct W8A8GemmArgs {
  uint32_t struct_size;
  int32_t epilogue;
  const int8_t* a;
  int64_t lda;
  const int8_t* b;
  int64_t ldb;
  int64_t m;
  int64_t n;
  int64_t k;
  const float* row_scale;
  const float* col_scale;
  int64_t col_scale_stride;
  const void* bias;
  int32_t bias_dtype;
  int32_t out_dtype;
  const void* residual;
  int64_t ldr;
  const float* gate;
  const int32_t* gate_labels;
  int64_t ldg;
  void* out;
  int64_t ldc;
  void* workspace;
  int64_t workspace_bytes;
  const struct W8A8RopeEpilogue* rope;
  void* stream;
} W8A8GemmArgs;

int w8a8_gemm(const W8A8GemmArgs* args);

/*
 * w8a8_gemm that allocates nothing and takes no workspace. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The split-K partials go to a file-scope device array of
 * W8A8_GEMM_SCRATCH_BYTES per GPU, which the library holds until the process
 * ends; a shape whose split needs more runs unsplit (the same result, more
 * slowly). A non-NULL args->workspace or a non-zero workspace_bytes is
 * rejected (W8A8_ERR_INVALID). Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (e.g. on two streams) race.
 * Nothing in the array needs clearing: every split writes its whole partial
 * tile before the reduction reads it. Otherwise identical to w8a8_gemm (same
 * arguments, numerics and errors).
 */
#define W8A8_GEMM_SCRATCH_BYTES (64ll << 20)
int w8a8_gemm_noalloc(const W8A8GemmArgs* args);

/*
 * Workspace bytes w8a8_gemm would use for an m x n x k GEMM on the current
 * device (0: the shape does not split K). No counterpart in the reference
 * (its int_mm calls a vendor GEMM that manages its own workspace); it lets
 * the caller allocate the split-K scratch once.
 */
int64_t w8a8_gemm_workspace_size(int64_t m, int64_t n, int64_t k);

/*
 * Standalone dequantization of an int32 accumulator (the epilogue of
 * w8a8_gemm without the GEMM).
 * Replaces: patches/parallel_int8.py:53-69 (dequantize),
 *           patches/tilelang_column_epilogue.py:10-40 (dequantize),
 *           patches/dit_column_linear.py:24-37 (_dequantize_eager).
 * acc: [m, n] int32, row stride ldacc. Other fields as in W8A8GemmArgs.
 */
typedef struct W8A8DequantArgs {
  uint32_t struct_size;
  int32_t epilogue;   /* W8A8_EPI_ROW or W8A8_EPI_COLUMN */
  const int32_t* acc;
  int64_t ldacc;
  int64_t m;
  int64_t n;
  const float* row_scale;
  const float* col_scale;
  int64_t col_scale_stride;
  const void* bias;
  int32_t bias_dtype;
  int32_t out_dtype;
  const void* residual;
  int64_t ldr;
  const float* gate;
  const int32_t* gate_labels;
  int64_t ldg;
  void* out;
  int64_t ldc;
  void* stream;
} W8A8DequantArgs;

int w8a8_dequantize(const W8A8DequantArgs* args);

/* ABI version (W8A8_ABI_VERSION). */
int w8a8_abi_version(void);

/* sizeof of each argument struct, by index: 0 Quant, 1 Swiglu, 2 Gemm,
 * 3 Dequant, 4 Norm, 5 RmsRope, 6 AttnPrepare, 7 Attention; -1 for an
 * unknown index. Lets bindings verify their layout. */
int64_t w8a8_struct_size(int32_t which);

/* Message describing the last error returned on the calling thread. */
const char* w8a8_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_H */
