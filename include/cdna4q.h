/*
 * cdna4q — quantized linear kernels for AMD Instinct MI355X (gfx950).
 *
 * Plain C ABI over HIP. Every entry point:
 *   - takes device pointers, element strides ("ld" = distance between rows,
 *     in elements) and sizes; tensors are row-major, K is the contiguous
 *     (reduction) dimension of both GEMM operands ("NT": D = A @ B^T with B
 *     stored [N, K], the nn.Linear weight layout);
 *   - enqueues asynchronously on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronizes, allocates device memory or frees it;
 *     all buffers belong to the caller;
 *   - returns C4Q_OK (0) or a negative status; c4q_last_error() then holds a
 *     message (thread-local). Invalid arguments are rejected before anything
 *     is enqueued.
 *
 * Layout contract of the fast (MFMA-tiled) kernels: base pointers 16-byte
 * aligned, row strides a multiple of 16 bytes, K a multiple of 16. Calls
 * outside it are still computed, bit-identically where the result is
 * integer/byte exact, by shape-agnostic fallback kernels.
 *
 * Each declaration names the reference (luix93/ComfyUI-AppleSilicon-Optimized)
 * interface it replaces, as path:line under that repository.
 */
#ifndef CDNA4Q_H
#define CDNA4Q_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define C4Q_ABI_VERSION 1

/* status codes */
#define C4Q_OK 0
#define C4Q_ERR_ARG (-1)          /* null pointer, bad enum value          */
#define C4Q_ERR_SHAPE (-2)        /* negative size, stride smaller than row */
#define C4Q_ERR_HIP (-4)          /* HIP launch / runtime error             */
#define C4Q_ERR_UNSUPPORTED (-5)  /* valid but unsupported combination      */

/* element types of floating-point tensors */
#define C4Q_BF16 0
#define C4Q_F16 1
#define C4Q_F32 2

/* scale layouts of c4q_f8_gemm_nt_scaled */
#define C4Q_SCALE_NONE 0
#define C4Q_SCALE_TENSOR 1   /* one fp32 value                         */
#define C4Q_SCALE_VECTOR 2   /* scale_a: [M] (rows); scale_b: [N] (cols) */

const char* c4q_last_error(void);
int c4q_abi_version(void);

/* C[M,N] int32 = A[M,K] int8 @ B[N,K]^T int8, exact.
 * Replaces i8_matmul2d_nt (_patches/int8_ext/int8_gemm.mm:1655-1703), the
 * kernel behind the torch._int_mm seam (_patches/int_mm_mps.py:90-110). */
int c4q_i8_gemm_nt_i32(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                       int32_t* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                       void* stream);

/* D[M,N] bf16 = bf16(f32(A@B^T) * row_scale[m]) [then bf16(D + bias[n])].
 * row_scale: fp32 [M]; bias: bf16 [N] or NULL.
 * Replaces i8_matmul2d_nt_fused (_patches/int8_ext/int8_gemm.mm:1709-1774). */
int c4q_i8_gemm_nt_fused(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                         uint16_t* d, int64_t ldd, const float* row_scale,
                         const uint16_t* bias, int64_t M, int64_t N, int64_t K,
                         void* stream);

/* D[M,N] bf16 = bf16(f32(A@B^T) * (col_scale[n] * row_scale[m])) [+ bias].
 * Replaces i8_matmul2d_nt_fused_cs (_patches/int8_ext/int8_gemm.mm:1823-1954);
 * its schedule switches (split_tail, long_schedule, moss_schedule) change no
 * output byte and have no counterpart here. */
int c4q_i8_gemm_nt_fused_cs(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                            uint16_t* d, int64_t ldd, const float* row_scale,
                            const float* col_scale, const uint16_t* bias,
                            int64_t M, int64_t N, int64_t K, void* stream);

/* fp16 variant: D[M,N] half = half(f32(A@B^T) * (col_scale[n] * row_scale[m]))
 * [then half(f32(D) + f32(bias[n]))], bias: fp16 [N] or NULL.
 * Replaces i8_matmul2d_nt_fused_cs_half (_patches/int8_ext/int8_gemm.mm:1965-2010,
 * epilogue nax_frag_store_dequant_cs_half :1161-1183), called by the Wan and
 * MiniMax-VAE INT8 projections (_patches/wan_fp16.py:40-42,
 * _patches/minimax_vae_int8.py:71-73). */
int c4q_i8_gemm_nt_fused_cs_f16(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                uint16_t* d, int64_t ldd, const float* row_scale,
                                const float* col_scale, const uint16_t* bias,
                                int64_t M, int64_t N, int64_t K, void* stream);

/* H3 QKV variant: the c4q_i8_gemm_nt_fused_cs bf16 result [M, 3*H*D] stored
 * straight into the attention layout: column n = kind*H*D + h*D + d goes to
 * out_kind[((h * M) + m) * D + d], out_0/1/2 = q/k/v, each [1, H, M, D]
 * contiguous. D must be a multiple of 8. Replaces i8_matmul2d_nt_fused_cs_qkv
 * (_patches/int8_ext/int8_gemm.mm:2028-2110, epilogue :445-474) behind
 * _int8_qkv_prequant (_patches/int8_linear_kernel_mps.py:266-360). */
int c4q_i8_gemm_nt_fused_cs_qkv(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                uint16_t* q, uint16_t* k, uint16_t* v, const float* row_scale,
                                const float* col_scale, const uint16_t* bias, int64_t M,
                                int64_t K, int64_t H, int64_t D, void* stream);

/* H3 QKV + Q/K RMSNorm + partial split-half RoPE, D = 128: the QKV variant
 * above, with each Q and K head row x (bf16 projection values) stored as
 *   inv = 1/sqrt(sum(x^2)/128 + eps), y = bf16((x*inv)*w)  w: q_weight/k_weight f32[128]
 *   d < 2R: bf16(bf16(f[r]*y_d) + f[1-r]*y_partner), f = freqs[m, d mod R, r, 0..1],
 *           r = (d >= R), partner = d+R or d-R;  d >= 2R: y_d
 * and V stored unchanged. freqs: bf16 [M, R, 2, 2], 4-byte aligned (may be
 * NULL when R = 0); 0 <= 2R <= 128. Q, K, V and the weights 16-byte
 * aligned. Replaces i8_matmul2d_nt_fused_cs_qkv_rms_rope
 * (_patches/int8_ext/int8_gemm.mm:2111-2209, kernel :683-861) behind
 * int8_qkv_rms_rope_prequant (_patches/int8_linear_kernel_mps.py:423-432). */
int c4q_i8_gemm_nt_fused_cs_qkv_rms_rope(const int8_t* a, int64_t lda, const int8_t* b,
                                         int64_t ldb, uint16_t* q, uint16_t* k, uint16_t* v,
                                         const float* row_scale, const float* col_scale,
                                         const uint16_t* bias, const uint16_t* freqs,
                                         const float* q_weight, const float* k_weight,
                                         int64_t M, int64_t K, int64_t H, int64_t R, float eps,
                                         void* stream);

/* H3 runtime-LoRA partition, D = 128: one of Q (kind 0), K (1) or V (2),
 * i.e. the partition's H*128 weight rows b, projected and stored as
 * out[1, H, M, 128] like the QKV scatter, with a bf16 low-rank delta
 * [M, H*128] (rows contiguous, 8-byte aligned) added after the bias:
 *   sd = bf16(f32(delta[m,n]) * f32(bf16(delta_scale))), value = bf16(value + sd)
 * then, for Q and K, the RMSNorm + partial RoPE of the variant above with
 * norm_weight f32[128] (16-byte aligned) and freqs bf16 [M, R, 2, 2].
 * out 16-byte aligned. Replaces i8_matmul2d_nt_fused_cs_qkv_lora_part
 * (_patches/int8_ext/int8_gemm.mm:2211-2330, kernels :915-1085) behind
 * _int8_qkv_prequant's runtime-LoRA route
 * (_patches/int8_linear_kernel_mps.py:351-379). */
int c4q_i8_gemm_nt_fused_cs_qkv_lora_part(const int8_t* a, int64_t lda, const int8_t* b,
                                          int64_t ldb, uint16_t* out, const float* row_scale,
                                          const float* col_scale, const uint16_t* bias,
                                          const uint16_t* delta, const uint16_t* freqs,
                                          const float* norm_weight, int64_t M, int64_t K,
                                          int64_t H, int64_t R, int kind, float delta_scale,
                                          float eps, void* stream);

/* Rowwise int8 activation quant of x[M,K] (bf16 or f16):
 * q[M,K] int8 and scales[M] fp32, bit-exact with comfy_kitchen
 * quantize_int8_rowwise. Replaces i8_quant_rowwise
 * (_patches/int8_ext/int8_gemm.mm:2332-2373, arithmetic :1337-1381). */
int c4q_i8_quant_rowwise(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                         float* scales, int64_t M, int64_t K, void* stream);

/* Fused attention head merge + ConvRot rotation + rowwise int8 quant:
 * x [B,H,S,D] bf16 contiguous -> q [B*S, H*D] int8 (row (b,s), column h*D+d)
 * and scales [B*S] fp32. rotate != 0: each 256-element group of a row is
 * rotated by the radix-4 Walsh-Hadamard butterflies of the reference kernel,
 * times 2^-4, rounded to bf16; rotate == 0: gather only. The quant is the
 * c4q_i8_quant_rowwise arithmetic. Needs 0 < D <= 256, H*D a multiple of 256
 * and at most 15360. Replaces i8_merge_rot_quant
 * (_patches/int8_ext/int8_gemm.mm:2545-2585, kernel :1429-1507), called by
 * int8_o_proj_prequant (_patches/int8_linear_kernel_mps.py:436-535). */
int c4q_i8_merge_rot_quant(const uint16_t* x, int64_t B, int64_t H, int64_t S, int64_t D,
                           int rotate, int8_t* q, float* scales, void* stream);

/* SwiGLU + ConvRot pre-pass of an INT8 fc2: x [M, 2F] bf16 contiguous
 * (gate columns [0,F), up columns [F,2F)), F a multiple of 256 ->
 * rot [M, F] bf16 contiguous, act = bf16(f32(silu_table[a]) * f32(b))
 * rotated per 256-element group as in c4q_i8_merge_rot_quant. silu_table:
 * 65,536 bf16 entries (SiLU of every bf16 value). x and rot 16-byte aligned.
 * Replaces i8_swiglu_rot (_patches/int8_ext/int8_gemm.mm:2593-2631, kernel
 * :1521-1554), called by the INT8 fc2 path (_patches/int8_linear_kernel_mps.py:756-770). */
int c4q_i8_swiglu_rot(const uint16_t* x, int64_t M, int64_t F, const uint16_t* silu_table,
                      uint16_t* rot, void* stream);

/* SwiGLU + ConvRot + rowwise quant in one pass: x [M, 2F] bf16 (16-byte
 * aligned) -> q [M, F] int8 contiguous and scales [M] fp32, the bytes of
 * c4q_i8_quant_rowwise(c4q_i8_swiglu_rot(x)); F a multiple of 256, at most
 * 15360. Replaces the reference bridge's i8_swiglu_rot_max_inplace_bf16 +
 * i8_quant_rowwise_premax_strided_bf16 pair (_patches/int8_ext/int8_gemm.mm:1249-1330). */
int c4q_i8_swiglu_rot_quant(const uint16_t* x, int64_t M, int64_t F, const uint16_t* silu_table,
                            int8_t* q, float* scales, void* stream);

/* H3 FC1/SwiGLU/FC2 bridge, front half: FC2's ConvRot-rotated, rowwise-
 * quantized activation from FC1's int8 input. Per chunk of tile_rows rows:
 * wide = c4q_i8_gemm_nt_fused_cs(a rows, w1 [W, K], row_scale rows,
 * col_scale [W], bias [W] or NULL) as bf16 [rows, W], F = W/2 a multiple
 * of 256; then q rows [rows, F] int8 and scales rows =
 * c4q_i8_swiglu_rot_quant(wide) (F <= 15360), or c4q_i8_swiglu_rot into rot
 * [rows, F] followed by c4q_i8_quant_rowwise (wider F). wide (tile_rows x W
 * bf16) and rot (tile_rows x F bf16; may be NULL when F <= 15360) are the
 * caller's scratch, 16-byte aligned; q [M, F] contiguous, scales [M]. Replaces
 * i8_mlp_bridge_prequant (_patches/int8_ext/int8_gemm.mm:2377-2537) behind
 * int8_mlp_bridge (_patches/int8_linear_kernel_mps.py:538-673). */
int c4q_i8_mlp_bridge_prequant(const int8_t* a, int64_t lda, const int8_t* w1, int64_t ldw,
                               const float* row_scale, const float* col_scale,
                               const uint16_t* bias, const uint16_t* silu_table, int64_t M,
                               int64_t K, int64_t W, int64_t tile_rows, uint16_t* wide,
                               uint16_t* rot, int8_t* q, float* scales, void* stream);

/* Bytes of the per-GPU device array that c4q_i8_mlp_bridge_prequant_noalloc
 * stages FC1 rows in (64 MiB, held by each GPU the library runs on until the
 * process ends). */
#define C4Q_BRIDGE_SCRATCH_BYTES (64ll << 20)

/* c4q_i8_mlp_bridge_prequant without caller scratch and without any device
 * allocation: FC1's bf16 rows (and, for F > 15360, their rotated halves) are
 * staged in the library's own C4Q_BRIDGE_SCRATCH_BYTES array on the current
 * device, in chunks of as many whole 128-row blocks as fit (all M rows at
 * once when they fit). Same outputs q [M, F] int8 and scales [M] fp32, byte
 * for byte, as c4q_i8_mlp_bridge_prequant. Rejects (C4Q_ERR_SHAPE) an F whose
 * 128-row chunk does not fit the array (F > 87381). Calls on one GPU share
 * its array: calls that overlap in time on one GPU (different streams, or
 * different host threads without ordering) race on it.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int c4q_i8_mlp_bridge_prequant_noalloc(const int8_t* a, int64_t lda, const int8_t* w1,
                                       int64_t ldw, const float* row_scale,
                                       const float* col_scale, const uint16_t* bias,
                                       const uint16_t* silu_table, int64_t M, int64_t K,
                                       int64_t W, int8_t* q, float* scales, void* stream);

/* torch._scaled_mm fp8 route: D[M,N] = out_dtype(((f32(A@B^T) * scale_a)
 * * scale_b) * scale_result + f32(bias[n])). A [M,K] and B [N,K] are e4m3fn
 * bytes; scale_result and bias may be NULL.
 * Replaces fp8fp8_matmul2d_nt (_patches/fp8_ext/fp8_matmul2d.mm:229-265)
 * together with the fp32 scale/bias tail of _fast_route
 * (_patches/scaled_mm_fp8.py:123-146). */
int c4q_f8_gemm_nt_scaled(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb,
                          void* d, int d_dtype, int64_t ldd,
                          const float* scale_a, int scale_a_mode,
                          const float* scale_b, int scale_b_mode,
                          const float* scale_result, const void* bias, int bias_dtype,
                          int64_t M, int64_t N, int64_t K, void* stream);

/* Dynamic per-tensor e4m3fn quant of n contiguous elements (bf16/f16):
 * scale[0] = amax/448 (1 if the tensor is all zeros), q = e4m3fn(clamp(x /
 * scale, +-448)). amax_ws: one fp32 of caller scratch.
 * The caller side of torch._scaled_mm; the clamp-then-cast follows
 * comfy_kitchen quantize_per_tensor_fp8 (_patches/comfykitchen_fp8.py:91-97). */
int c4q_f8_quant_pertensor(const void* x, int x_dtype, int64_t n, uint8_t* q,
                           float* scale, float* amax_ws, void* stream);

/* out[n] = T(decode(w[n]) * T(scale[0])) for T = out_dtype (bf16/f16); the
 * plain exact decode when scale is NULL. Replaces comfy_kitchen
 * dequantize_per_tensor_fp8 (_patches/comfykitchen_fp8.py:86-89) and
 * decode_fp8 (_patches/_common.py:249-273). */
int c4q_fp8_dequant(const uint8_t* w, int64_t n, const float* scale, void* out,
                    int out_dtype, void* stream);

/* W8A16 linear: D[M,N] = out_dtype(A@W'^T + f32(bias[n])) with
 * A [M,K] bf16 or f16 and W [N,K] e4m3fn dequantized in registers to the
 * activation type, W' = T(decode(W) * T(w_scale[0])) (w_scale NULL = plain
 * decode). act_table (bf16 output only, or NULL): 65,536 bf16 entries applied
 * to the rounded output (e.g. GELU-tanh for an MLP up-projection).
 * M <= 32 (decode shapes, K <= 4096, aligned operands) takes a split-K route
 * that streams W at memory bandwidth, M <= 64 with N <= 12288 two passes of
 * it over the row halves; larger M the MFMA-tiled route.
 * Replaces w8a16_bias_bf16 / w8a16_f32
 * (_patches/fp8s_ext/w8a16_gemm.mm:286-314) behind _w8a16_forward
 * (_patches/linear_fp8_w8a16.py:151-196). */
int c4q_w8a16_gemm_nt(const void* a, int a_dtype, int64_t lda, const uint8_t* w, int64_t ldw,
                      const float* w_scale, void* d, int d_dtype, int64_t ldd,
                      const void* bias, int bias_dtype, const uint16_t* act_table,
                      int64_t M, int64_t N, int64_t K, void* stream);

/* Fused gate/up FFN pair, bf16 out [M, N_out]:
 *   x1 = bf16(f32(A@Wg^T) * (gate_scale[c] * row_scale[m]))
 *   x2 = bf16(f32(A@Wu^T) * (up_scale[c] * row_scale[m]))
 *   D  = bf16(f32(T1[x1]) * f32(T2[x2]))   (NULL table = identity)
 * Wg, Wu: int8 [N_out, K] with row stride ldw. Krea2 SwiGLU: T1 = SiLU
 * table, T2 = NULL. MOSS FC1/SiTU: Wg/Wu = the hidden/gate halves of one
 * [2F, K] weight, T1/T2 = its SiTU tables.
 * Replaces pair_128_128_4_4_0 (_patches/krea2_ffn_pair.metal:281-304) and
 * fc1_situ (_patches/moss_ffn_mps.metal:278-301). */
int c4q_i8_ffn_pair(const int8_t* a, int64_t lda, const int8_t* w_gate, const int8_t* w_up,
                    int64_t ldw, uint16_t* d, int64_t ldd, const float* row_scale,
                    const float* gate_scale, const float* up_scale,
                    const uint16_t* table_gate, const uint16_t* table_up,
                    int64_t M, int64_t N_out, int64_t K, void* stream);

/* bf16 fused FC1/SiTU pair, bf16 out [M, N_out]:
 *   h = bf16(f32(A@Wh^T)),  g = bf16(f32(A@Wg^T))   (fp32 accumulation)
 *   D = bf16(f32(T_h[h]) * f32(T_g[g]))              (NULL table = identity)
 * A [M,K] bf16; Wh, Wg [N_out, K] bf16 with row stride ldw: the hidden and
 * gate halves of one [2F, K] weight; T_h / T_g the SiTU tables (65,536 bf16).
 * Replaces moss_64_128_2_4_0 (_patches/moss_bf16_ffn_pair.metal:282-304)
 * behind project() (_patches/moss_bf16_ffn_pair.py:36-48). */
int c4q_bf16_ffn_pair(const uint16_t* a, int64_t lda, const uint16_t* w_hidden,
                      const uint16_t* w_gate, int64_t ldw, uint16_t* d, int64_t ldd,
                      const uint16_t* table_hidden, const uint16_t* table_gate,
                      int64_t M, int64_t N_out, int64_t K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CDNA4Q_H */
