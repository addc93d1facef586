/*
 * diffucore_amd: C ABI of the MI355X (gfx950) quantized denoiser hot path.
 *
 * The reference (nawka12/diffucore) binds this path from Python: Triton
 * kernels and torch ops in src/diffucore/models/_int8.py, and two pybind11
 * extension modules built by torch.utils.cpp_extension,
 * src/diffucore/kernels/int8_attn_sm80.cu (fwd) and
 * src/diffucore/kernels/int8_gemm_sm75.cu (scaled_mm). Each entry point below
 * names the reference interface it replaces.
 *
 * Conventions (all entry points):
 *  - Plain C types only. Device pointers are raw HIP device addresses.
 *  - `stream` is a hipStream_t (NULL = the null stream). Every entry point only
 *    enqueues work on `stream`; none synchronizes and none allocates memory.
 *  - Return 0 on success, else one of DC_E*; dc_last_error() then holds a
 *    thread-local message.
 *  - dtype codes: DC_F16, DC_BF16, DC_F32, DC_I32 (GEMM output only).
 *  - Work runs on the calling thread's current HIP device.
 */
#ifndef DIFFUCORE_AMD_H
#define DIFFUCORE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { DC_F16 = 0, DC_BF16 = 1, DC_F32 = 2, DC_I32 = 3, DC_NONE = -1 };
enum { DC_OK = 0, DC_EINVAL = 1, DC_EUNSUPPORTED = 2, DC_EHIP = 3, DC_EWORKSPACE = 4 };

/* Message for the last failing call on this thread ("" if none). */
const char* dc_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int dc_abi_version(void);

/*
 * Per-row int8 activation quantization, optionally after the ConvRot rotation.
 * Replaces quantize_activation (src/diffucore/models/_int8.py:299-310), i.e.
 * the Triton _rot_quant_kernel (_int8.py:399-406) and its torch fallback
 * _quantize_rows(_rotate(x.float(), group)) (_int8.py:87-97, 79-84).
 *
 *   x      [M, K] of x_dtype (DC_F16/DC_BF16/DC_F32), row stride ldx elements
 *   group  0 (none) or 256 (x @ H_256 per 256-wide group; needs K % 256 == 0)
 *   q      [M, K] int8 out, row stride ldq bytes
 *   scale  [M] float32 out: max(amax / 127, 1e-30)
 * Codes are clamp(rint(x / scale), -128, 127) with an IEEE float32 division.
 */
int dc_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int group,
                     int8_t* q, int64_t ldq, float* scale, void* stream);

/* Activations for dc_act_quantize_rows. */
enum { DC_ACT_NONE = 0, DC_ACT_GELU_ERF = 1, DC_ACT_GELU_TANH = 2, DC_ACT_GEGLU = 3 };

/*
 * dc_quantize_rows of the rows of concat(x1, act(x2)), in one pass:
 *   x1 [M, K1] row stride ld1 (may be NULL with K1 == 0), taken as it is;
 *   x2 [M, K2] row stride ld2, through act: GELU computed in float32 and
 *   rounded to x_dtype (DC_F16 or DC_BF16), the dtype of both inputs;
 *   q [M, K1 + K2] int8 (row stride ldq), scale [M] as dc_quantize_rows.
 * K1 and K2 are multiples of 256, K1 + K2 <= 32768; 16-byte aligned rows.
 * Replaces the reference's fused MLP middle, GEMM1 output -> GELU -> l2's
 * ConvRot + quantize in one row pass (src/diffucore/models/_int8.py:326-358,
 * 419-443: _gelu_quantize / _gelu_f16_rot_quant_kernel); act =
 * DC_ACT_GELU_TANH covers FLUX's MLP middle (flux_dit.py:228-239) and, with
 * x1, its single-block linear2 input cat(attention, gelu_tanh(mlp))
 * (flux_dit.py:335), which the reference builds with torch ops before
 * quantizing.
 * act = DC_ACT_GEGLU: x2 rows are [M, 2 K2] (row stride ld2 >= 2 K2), the
 * value half then the gate half of a GEGLU projection, and the K2 columns fed
 * to the quantizer are round(value * round(gelu_erf(gate))) (the SD1.5 / SDXL
 * UNet's GEGLU, src/diffucore/models/unet.py:148-155: x * F.gelu(gate) on the
 * two chunks of proj's output, each op rounded to x_dtype).
 */
int dc_act_quantize_rows(const void* x1, int64_t ld1, int64_t K1, const void* x2, int64_t ld2, int64_t K2,
                         int act, int x_dtype, int64_t M, int group, int8_t* q, int64_t ldq, float* scale,
                         void* stream);

/*
 * dc_quantize_rows of the rows of y = round(LayerNorm(x) * sc1 + shift), in one
 * pass: LayerNorm without affine weights in float32 (mean, then the centered
 * variance, rstd = 1 / sqrt(var + eps)), y in float32 with separate roundings,
 * rounded to mod_dtype (DC_F16 or DC_BF16) before the rotation and the codes.
 *   x [M, K] of x_dtype (mod_dtype or DC_F32), row stride ldx;
 *   sc1 (the caller's 1 + scale) and shift: row m / rows_per_mod of [*, K]
 *   arrays of mod_dtype, row stride ldm (rows_per_mod rows share one row, e.g.
 *   the tokens of one sample);
 *   q [M, K] int8 (row stride ldq), scale [M] as dc_quantize_rows.
 * K % 256 == 0, K <= 32768, 16-byte aligned rows.
 * Replaces the reference's LayerNorm-modulate glue (src/diffucore/models/
 * _fused.py:73-85 _ln_mod_kernel, ln_mod :151-156; eager in flux_dit.py's
 * blocks) followed by quantize_activation in the next Int8Linear: the
 * modulated rows are never written out.
 */
int dc_ln_mod_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* sc1,
                            const void* shift, int mod_dtype, int64_t ldm, int64_t rows_per_mod, float eps,
                            int group, int8_t* q, int64_t ldq, float* scale, void* stream);

/* Flags of dc_qk_norm_rope. */
enum {
  DC_QK_ROPE_HALF = 1,   /* rotary pairs (i, i + D/2) (Anima); otherwise (2i, 2i + 1) (FLUX) */
  DC_QK_WEIGHT_F32 = 2   /* n = round(w * (x * rrms)) (Anima); otherwise round(round(x * rrms) * w) (FLUX) */
};

/*
 * Per-head RMSNorm of q and k, then the rotary embedding, in one pass; also
 * copies v when given (to gather several streams' v into one buffer).
 *   q, k, v       [B, L, H, D] of dtype (DC_F16 or DC_BF16), element strides
 *                 {b, l, h} in *_strides, D contiguous; k and v may be NULL;
 *   *_out         [B, L, H, D] outputs, strides in *_out_strides (may alias
 *                 the input with the same strides);
 *   q/k_weight    [D] of weight_dtype (dtype or DC_F32);
 *   rrms          rsqrt(sum(x^2) / D + eps), x^2 and the sum in float32;
 *   freqs         float32 [.., L, D/2, 2, 2] rotary matrices, position l of
 *                 sample b at freqs + b * freqs_batch_stride + l *
 *                 freqs_pos_stride; NULL for no rotary embedding. A pair
 *                 (a, b) becomes (round(f00 a + f01 b), round(f10 a + f11 b)),
 *                 each product and sum rounded to float32 on its own.
 * D in {32, 64, 128, 256}; 16-byte aligned rows and tables.
 * Replaces FLUX's QKNorm + apply_rope (src/diffucore/models/flux_dit.py:
 * 129-151, 179-184; eager torch ops) with flags 0, and Anima's
 * qk_norm_rope (_fused.py:114-139, 174-185) with DC_QK_ROPE_HALF |
 * DC_QK_WEIGHT_F32.
 */
int dc_qk_norm_rope(int dtype, int64_t B, int64_t L, int64_t H, int64_t D, int flags, float eps,
                    const void* q, const int64_t* q_strides, const void* q_weight,
                    const void* k, const int64_t* k_strides, const void* k_weight, int weight_dtype,
                    const float* freqs, int64_t freqs_batch_stride, int64_t freqs_pos_stride,
                    void* q_out, const int64_t* q_out_strides, void* k_out, const int64_t* k_out_strides,
                    const void* v, const int64_t* v_strides, void* v_out, const int64_t* v_out_strides,
                    void* stream);

/*
 * W8A8 GEMM on int8 MFMA with int32 accumulation and a fused epilogue.
 *   a   [M, K] int8 (activations), row stride lda
 *   w   [N, K] int8 (nn.Linear weight layout), row stride ldw
 * out_dtype == DC_I32: out = a @ w.T as int32 (sx, sw, bias ignored).
 *   Replaces int_mm (src/diffucore/models/_int8.py:200-207), torch._int_mm.
 * out_dtype in {DC_F16, DC_BF16, DC_F32}:
 *   out[m, n] = cast(float(acc[m, n]) * (sx[m] * sw[n])), then, when bias is
 *   given (bias_dtype != DC_NONE), out = cast(out + cast(bias[n])).
 *   Replaces scaled_mm (_int8.py:266-276; kernels/int8_gemm_sm75.cu:75-88)
 *   and int_mm + rescale (_int8.py:313-323), rounding bit for bit like them.
 * Needs K % 16 == 0, lda % 16 == 0, ldw % 16 == 0 and 16-byte aligned a, w.
 * workspace / ws_bytes (may be NULL / 0): scratch for split-K on problems
 * whose tiles would leave most of the device idle (small M, long K; see
 * dc_w8a8_gemm_workspace_bytes). The k range is split over workgroups that
 * write int32 partial sums there, and an epilogue pass adds them (exact) and
 * applies the same rescale, bias and cast: results are bit-identical to the
 * unsplit call. Without enough workspace the call runs unsplit.
 */
int dc_w8a8_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* sx,
                 const float* sw, const void* bias, int bias_dtype, void* out, int out_dtype,
                 int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes,
                 void* stream);

/*
 * Workspace bytes dc_w8a8_gemm uses for split-K on this problem on the
 * current device (0: it runs unsplit). No counterpart in the reference, whose
 * GEMMs are torch._int_mm and one CUTLASS kernel (_int8.py:200-276).
 */
size_t dc_w8a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw);

/*
 * Which GEMM kernel dc_w8a8_gemm runs for a problem on the current device:
 * one of the DC_GEMM_PLAN_* codes, or -1 for a shape it rejects. Tiles are
 * chosen by how full the last round of workgroups keeps the device. No
 * counterpart in the reference (its GEMMs come from torch._int_mm and one
 * CUTLASS configuration, _int8.py:200-276); for profiling and tests.
 */
enum {
  DC_GEMM_PLAN_256x256 = 0,      /* 8 waves, 128 x 64 wave tiles, register-staged loads */
  DC_GEMM_PLAN_192x256 = 1,      /* 8 waves, 96 x 64 wave tiles */
  DC_GEMM_PLAN_128x128 = 2,      /* 4 waves, 64 x 64 wave tiles, 2 workgroups per CU */
  DC_GEMM_PLAN_DMA_256x256 = 3,  /* 4 waves, 128 x 128 wave tiles, loads straight into LDS */
  DC_GEMM_PLAN_192x128 = 4       /* 192 (n) x 128 (m) on 4 waves, 96 x 64 wave tiles, 1 workgroup per CU */
};
int dc_w8a8_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw);

/*
 * Grouped W8A8 GEMM: up to DC_GEMM_MAX_GROUP problems that share N, K, the
 * output dtype and the bias dtype, each with its own activations, weights,
 * scales, bias and output, in one launch of the DMA-fed 256 x 256 kernel
 * (their tiles back to back in one grid). Each output is bit-identical to
 * dc_w8a8_gemm on the same problem. No counterpart in the reference, which
 * runs each Int8Linear on its own (_int8.py:158-167); it is for callers that
 * hold several independent linears of one shape at once, such as FLUX's
 * double-stream blocks (flux_dit.py:275-330: the img and txt streams' qkv,
 * proj and MLP-down layers), where a small problem's tiles then fill CUs the
 * large one leaves idle in its last round.
 * Needs K % 256 == 0 and, per problem, lda, ldw multiples of 16 with
 * 256 * lda and 256 * ldw below 2^31, 16-byte aligned a and w, ldo >= N.
 * Problems with M == 0 are skipped. No split-K: the workspace of dc_w8a8_gemm
 * has no counterpart here.
 */
#define DC_GEMM_MAX_GROUP 4
typedef struct dc_gemm_problem {
  const int8_t* a;     /* [M, K] int8, row stride lda */
  int64_t lda;
  const int8_t* w;     /* [N, K] int8, row stride ldw */
  int64_t ldw;
  const float* sx;     /* [M] row scales (ignored for DC_I32 output) */
  const float* sw;     /* [N] channel scales (ignored for DC_I32 output) */
  const void* bias;    /* [N] of bias_dtype, or NULL with DC_NONE */
  void* out;           /* [M, N] of out_dtype, row stride ldo */
  int64_t ldo;
  int64_t M;
} dc_gemm_problem;
int dc_w8a8_gemm_grouped(const dc_gemm_problem* problems, int count, int64_t N, int64_t K, int bias_dtype,
                         int out_dtype, void* stream);

/*
 * dc_w8a8_gemm_grouped with a gated residual in the epilogue: problem i's
 * output is res + gate * y, y being what dc_w8a8_gemm_grouped writes (scales,
 * bias, cast), rounded as torch rounds FLUX's two bf16 ops: t = round(gate[n]
 * * y[m, n]), out[m, n] = round(res[m, n] + t), each to out_dtype (DC_F16,
 * DC_BF16 or DC_F32), with no fused multiply-add. No counterpart in the
 * reference, whose FLUX blocks run the linear, then x + gate * out as two
 * torch ops (flux_dit.py:298-301, 336); it is for callers that apply such
 * a gate and residual to a W8A8 layer's output (FLUX's attention projection,
 * MLP down and single-block linear2), saving those two passes over [M, N].
 * gates[i].res is [M, N] of out_dtype with row stride ldr >= N; it may be
 * problem i's own output (in place, ldr == ldo) but must not overlap any
 * other output. gates[i].gate is one row of N values of out_dtype (the same
 * gate for every row). Same requirements as dc_w8a8_gemm_grouped otherwise.
 */
typedef struct dc_gemm_gate {
  const void* res;     /* [M, N] of out_dtype, row stride ldr */
  int64_t ldr;
  const void* gate;    /* [N] of out_dtype */
} dc_gemm_gate;
int dc_w8a8_gemm_grouped_gated(const dc_gemm_problem* problems, const dc_gemm_gate* gates, int count, int64_t N,
                               int64_t K, int bias_dtype, int out_dtype, void* stream);

/*
 * Whether one dc_w8a8_gemm_grouped launch over problems of these row counts
 * is expected to beat separate dc_w8a8_gemm calls on the current device: 1
 * when K % 256 == 0, there are at least two non-empty problems and their
 * 256 x 256 tiles together need no more rounds of the device's CUs than the
 * largest problem's alone; 0 otherwise; -1 for bad arguments. No counterpart
 * in the reference.
 */
int dc_w8a8_gemm_group_plan(const int64_t* Ms, int count, int64_t N, int64_t K);

/*
 * The rescale pass on an int32 accumulator, for callers that hold one.
 * Replaces rescale (src/diffucore/models/_int8.py:313-323) and the Triton
 * _rescale_kernel (_int8.py:408-417). Same rounding as dc_w8a8_gemm.
 */
int dc_rescale(const int32_t* acc, int64_t lda, const float* sx, const float* sw,
               const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
               int64_t M, int64_t N, void* stream);

/*
 * Workspace size in bytes for dc_int8_attn_fwd at this shape on the current
 * device. Replaces the scratch tensors fwd allocates itself
 * (src/diffucore/kernels/int8_attn_sm80.cu:469-476).
 */
size_t dc_int8_attn_workspace_bytes(int B, int H, int Lq, int Lk, int D);

/*
 * How dc_int8_attn_fwd splits its work at this shape on the current device
 * (no counterpart in the reference, whose grid is one CTA per 128-query tile,
 * int8_attn_sm80.cu:486-494; for profiling and tests). Head dims up to 64: the
 * 128-query tiles (b, h, tile) in that order fill whole rounds of the
 * device's resident workgroups, *dp_tiles of them, each run whole; the
 * remaining *sk_tiles tiles' (query tile, 64-key tile) pairs are shared by
 * *sk_blocks stream-K workgroups (0 when the last round is run whole) whose
 * partial results a merge kernel combines. Head dims above 64: 256-query
 * tiles, all run whole (*dp_tiles of them, *sk_blocks = *sk_tiles = 0), when
 * there are at least as many as the device has compute units and the key
 * range is at most 131072; otherwise the 128-query split above. Returns 0, or
 * DC_EINVAL for a bad shape or dtype.
 */
int dc_int8_attn_plan(int dtype, int B, int H, int Lq, int Lk, int D, int* dp_tiles, int* sk_blocks,
                      int* sk_tiles);

/*
 * INT8-QK / 16-bit-PV flash attention.
 * Replaces fwd(q, k, v, sm_scale) (src/diffucore/kernels/int8_attn_sm80.cu:460-497),
 * called from attention_blhd / attention_bhld (src/diffucore/models/_attention.py:216-217, 268-271).
 *   q [B, Lq, H, D], k and v [B, Lk, H, D], o [B, Lq, H, D], all of `dtype`
 *   (DC_F16 or DC_BF16), given as element strides for the (B, L, H) dims;
 *   D is contiguous. D % 8 == 0, D <= 128, strides % 8 == 0, 16-byte aligned.
 *   sm_scale: softmax scale (the reference passes D ** -0.5).
 * K is smoothed by its per-channel mean and quantized per 64-key block; Q is
 * quantized per token inside the attention kernel; S = Q K^T runs on int8
 * MFMA into int32; the online softmax is float32 in base 2; P V runs on
 * 16-bit MFMA with float32 accumulation. The workspace
 * (dc_int8_attn_workspace_bytes) holds, at 256-byte aligned offsets in order:
 *   k8    int8 [B, H, Lk64, Dp]   Lk64 = Lk rounded up to 64, Dp = 64 or 128
 *   ks    f32  [B, H, Lk64 / 64]  per-block scale amax / 127
 *   kpart f32  [B, H, ceil(Lk / 128), D]   per-window key sums
 *   ksum  f32  [B, H, D]                    per-channel key sums
 *   part  f32  [2 * sk_blocks][128 * Dp + 256]  stream-K partial results:
 *         unnormalized O [128][Dp], row maxima [128], row sums [128]
 */
int dc_int8_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                     int H, int Lq, int Lk, int D, const int64_t q_strides[3],
                     const int64_t k_strides[3], const int64_t v_strides[3],
                     const int64_t o_strides[3], float sm_scale, void* workspace,
                     size_t ws_bytes, void* stream);

/* Scratch bytes dc_int8_attn_fwd_noalloc holds on each GPU it runs on (64 MiB). */
#define DC_ATTN_NOALLOC_MAX_BYTES (64u << 20)

/*
 * dc_int8_attn_fwd without a workspace argument: the same kernels and work
 * split, with the workspace taken from a scratch array the library keeps in
 * device memory (DC_ATTN_NOALLOC_MAX_BYTES per GPU, held until the process
 * ends). No counterpart in the reference (whose fwd allocates its scratch
 * through torch, int8_attn_sm80.cu:469-476): it is for callers that cannot
 * allocate - code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. It calls no hipMalloc / hipFree. A call whose
 * workspace (dc_int8_attn_workspace_bytes) would exceed the scratch returns
 * DC_EWORKSPACE with a message (FLUX 1024^2 attention needs 14.7 MB). Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (two streams, two threads) race and must be ordered by the caller; calls in
 * one stream are ordered already. Nothing in the scratch needs to start at
 * zero (every byte a call reads, it wrote first). The first call on each
 * device looks up that device's scratch address (hipGetSymbolAddress): make
 * one call on a device before capturing calls on it into a HIP graph.
 */
int dc_int8_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                             int H, int Lq, int Lk, int D, const int64_t q_strides[3],
                             const int64_t k_strides[3], const int64_t v_strides[3],
                             const int64_t o_strides[3], float sm_scale, void* stream);

/*
 * The per-token Q quantizer of dc_int8_attn_fwd (the same device code), with
 * its codes written out for verification: q8 int8 [B, H, Lq32, Dp] and
 * qs f32 [B, H, Lq32] = amax / 127, Lq32 = Lq rounded up to 32; rows past Lq
 * and channels past D are 0. Replaces the Q prologue of the reference's
 * attn_kernel (src/diffucore/kernels/int8_attn_sm80.cu:341-388), which keeps
 * its codes in registers.
 */
int dc_int8_attn_quantize_q(const void* q, int dtype, int B, int H, int Lq, int D,
                            const int64_t q_strides[3], int8_t* q8, float* qs, void* stream);

/*
 * MFMA throughput calibration (no counterpart in the reference; measurement
 * only). Launches one workgroup per compute unit with `waves` (1 or 2) waves
 * per SIMD, each issuing `iters` x 8 independent back-to-back MFMAs on 4
 * accumulators: kind 0 v_mfma_i32_32x32x32_i8 (65536 ops each), kind 1
 * v_mfma_f32_32x32x16_bf16 (32768 flops each); vary = 1 cycles each wave
 * through 8 operand pairs of per-lane hashed values (uniform int8 codes, bf16
 * magnitudes in [0.5, 2)), vary = 0 reuses one pair. Writes one int per wave
 * to sink[units * 4 * waves] so the work is kept. The caller times the launch
 * on `stream`; dc_mfma_probe_units() gives the unit count. Returns 0,
 * DC_EINVAL or DC_EHIP.
 */
int dc_mfma_probe(int kind, int vary, int waves, int iters, int* sink, void* stream);
int dc_mfma_probe_units(void);

#ifdef __cplusplus
}
#endif

#endif /* DIFFUCORE_AMD_H */
