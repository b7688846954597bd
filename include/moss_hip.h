/*
 * libmoss_hip.so -- C-ABI of the MI355X (gfx950) INT4-G32 quantized-linear path.
 *
 * Conventions (mirroring the reference's native launch convention,
 * src/moss_tts/_runtime/attention_native.cu:91-97 and attention_native.py:26-44):
 *   - every pointer is a device pointer owned by the caller; nothing is allocated inside;
 *   - bf16 tensors are passed as raw 16-bit patterns, row-major and contiguous;
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream); launches are
 *     asynchronous on it and graph-capturable (no host sync, no allocation);
 *   - the return value is a hipError_t (0 = success); argument errors return
 *     hipErrorInvalidValue (1) before anything is launched.
 *
 * Row-packed INT4-G32 weight ("rowpack", per output row n, G = K/32 groups):
 *   qw  uint32 [N, K/8]  group g = words 4g..4g+3; word j covers k = 32g+8j+t, the code of
 *                        t = 2i at bits [4i,4i+4), of t = 2i+1 at bits [16+4i,20+4i)
 *   sc  bf16   [N, G]
 *   zp  uint8  [N, G/2]  blocks of 128 groups: for block c (r = min(128, G-128c) groups)
 *                        byte 64c+b = z[128c+b] | z[128c+r/2+b] << 4
 *   w[n,k] = bf16_rne(float(q - z) * float(s))
 * The GEMVs' exact mode and the GEMMs form that value in registers from (128+q)*s - (128+z)*s in
 * fp32, exact for every scale below 2^120 (subnormal scales included); moss_w4g32_dequant_bf16 is
 * exact for every finite scale.  The Python loaders reject scales at or above 2^120.
 */
#ifndef MOSS_HIP_H
#define MOSS_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- library */
int moss_abi_version(void);
const char *moss_error_string(int code);
/* 0 if the current device is gfx950; writes its gcnArchName into arch_out.
 * Replaces the SM90 capability check of src/moss_tts/api.py:79-80. */
int moss_check_device(char *arch_out, int arch_len);

/* ------------------------------------------------------- INT4-G32 weights */
/* AutoGPTQ-style qweight int32 [K/8,N], scales bf16 [K/32,N], qzeros int32 [K/32,N/8]
 * (zero points stored literally) -> rowpack.  Replaces the install-time repack of
 * src/moss_tts/_runtime/dp4a_packing.py:128-160 (pack_interleaved :15-19). */
int moss_w4g32_repack_gptq(const void *qweight, const void *scales, const void *qzeros, void *qw, void *sc,
                           void *zp, int K, int N, void *stream);

/* The reference's calibrated export (packed u8 [N,K/2], two's-complement nibbles, byte j =
 * codes 2j | 2j+1 << 4) -> rowpack codes q = u ^ 8 and zeros z = 8 (the caller copies the
 * bf16-exact scales).  Replaces install_calibrated's buffers,
 * src/moss_tts/_runtime/calibrated_backend.py:30-56 (format: src/moss_tts/calibration.py:190-203). */
int moss_w4g32_import_signed(const void *packed, void *qw, void *zp, int K, int N, void *stream);

/* rowpack -> unsigned codes u8 [N,K].  Counterpart of unpack_signed,
 * src/moss_tts/_runtime/calibrated_backend.py:8-13. */
int moss_w4g32_unpack_codes(const void *qw, void *codes, int K, int N, void *stream);

/* rowpack -> bf16 [N,K], bit-exact dequant.  Counterpart of dequantize,
 * src/moss_tts/_runtime/calibrated_quant.py:41-42. */
int moss_w4g32_dequant_bf16(const void *qw, const void *sc, const void *zp, void *w, int K, int N, void *stream);

/* fp32 [N,K] -> rowpack with the asymmetric min-max RTN quantizer per (row, 32-group).
 * The synthetic-weight recipe; role of static_scales + quantization,
 * src/moss_tts/_runtime/calibrated_quant.py:36-38. */
int moss_w4g32_quantize_minmax(const void *w, void *qw, void *sc, void *zp, int K, int N, void *stream);

/* fp32 [N,K] -> rowpack with the reference's static symmetric scales and round-to-nearest codes:
 * s = bf16(max(max|w_g|, 1e-8) / 7) per (row, 32-group), c = clamp(rint(w / s), -7, 7) (IEEE
 * division, ties to even), stored as q = c + 8 with z = 8 (so the dequant is bf16(c * s)).
 * static_scales and the no-Hessian rounding of src/moss_tts/_runtime/calibrated_quant.py:36-38,74-77. */
int moss_w4g32_quantize_symmetric(const void *w, void *qw, void *sc, void *zp, int K, int N, void *stream);

/* ------------------------------------------------------------ decode GEMV */
/* dequant_mode of the decode GEMVs:
 *   MOSS_DEQUANT_EXACT (0)      every weight is the bit-exact bf16 dequant bf16_rne((q-z)*s)
 *                               (calibrated_quant.py:41-42) before it multiplies x; the
 *                               result is an fp32 dot of exactly the reference's dequantized
 *                               weights (default);
 *   MOSS_DEQUANT_UNROUNDED (1)  sum_g s * sum (q-z) x without the per-weight bf16 rounding
 *                               (about half the VALU work; error vs. the exact form bounded
 *                               by 2^-9 * sum |w x|). */
#define MOSS_DEQUANT_EXACT 0
#define MOSS_DEQUANT_UNROUNDED 1

/* y bf16 [M, N] = x bf16 [M, K] . dequant(W)^T, K % 64 == 0, K <= 16384.
 * M = 1: the decode GEMV; rows_per_wave in {0 (auto), 1, 2, 4}.
 * M = 2 .. 4 (MOSS_DEQUANT_EXACT only; K <= 4096 or K in {8192, 12288, 16384}): one pass over the
 * weights for all M tokens, every row of y bit-identical to the M = 1 GEMV of that token's x
 * (rows_per_wave is ignored).
 * Replaces the W4A8 projection linear() of src/moss_tts/_runtime/dp4a_scaled.py:81-95 (and
 * int4_dp4a, int4_dp4a.py:56-74). */
int moss_w4g32_gemv(const void *x, const void *qw, const void *sc, const void *zp, void *y, int M, int K, int N,
                    int rows_per_wave, int dequant_mode, void *stream);

/* Fused gate||up GEMV + SiLU*mul: W has 2*N_half rows (gate rows first, up rows second,
 * src/moss_tts/_runtime/llm.py:144); y bf16 [N_half] = bf16(bf16(silu(bf16(g))) * bf16(u)).
 * Replaces linear(..., paired=True) of src/moss_tts/_runtime/dp4a_scaled.py:64-68,81-95. */
int moss_w4g32_gateup_silu(const void *x, const void *qw, const void *sc, const void *zp, void *y, int M, int K,
                           int N_half, int rows_per_wave, int dequant_mode, void *stream);

/* Fused (add+)RMSNorm + decode GEMV: the projection's input is normalized inside the kernel
 * (each workgroup recomputes it into LDS while its weight loads are in flight).
 * res == NULL:  xn = rmsnorm(x) * norm_w;
 * res != NULL:  s = bf16(x + res) is stored to sum_out (which must not overlap x or res) and
 *               xn = rmsnorm(s) * norm_w.
 * Rounding points and summation order are those of moss_rmsnorm, so the normalized row is
 * bit-identical to moss_rmsnorm's, and for K <= 4096 the result is bit-identical to moss_rmsnorm
 * followed by moss_w4g32_gemv (at K = 8192 that GEMV splits K over two waves, and the two results
 * differ only by that fp32 summation order).  K % 2048 == 0, K <= 8192, M is 1.
 * Replaces the fused add+RMSNorm+quant+projection of
 * src/moss_tts/_runtime/dp4a_norm_projection.py:48-166 (and gateup_cluster.py:44-157). */
int moss_w4g32_norm_gemv(const void *x, const void *res, const void *norm_w, void *sum_out, float eps, const void *qw,
                         const void *sc, const void *zp, void *y, int K, int N, int rows_per_wave, int dequant_mode,
                         void *stream);

/* The same in front of the fused gate||up GEMV with the SiLU*mul epilogue (W has 2*N_half rows). */
int moss_w4g32_norm_gateup_silu(const void *x, const void *res, const void *norm_w, void *sum_out, float eps,
                                const void *qw, const void *sc, const void *zp, void *y, int K, int N_half,
                                int rows_per_wave, int dequant_mode, void *stream);

/* --------------------------------------------------- bf16-weight decode GEMV */
/* y bf16 [N] = bf16(sum_k f32(W[n,k]) * f32(x[k])), W bf16 [N, K] row-major (16-byte aligned), fp32
 * accumulate; K % 512 == 0, K / 512 in {1..8, 12, 16}; rows_per_wave in {0 (auto), 1, 2, 4}.  The
 * reference's bf16 decode projection: linear_decode / _gemv, src/moss_tts/_runtime/kernels.py:93-108,
 * and F.linear of the output heads, src/moss_tts/_runtime/llm.py:270-279. */
int moss_bf16_gemv(const void *x, const void *w, void *y, int K, int N, int rows_per_wave, void *stream);

/* The same behind the fused (add+)RMSNorm of moss_w4g32_norm_gemv (same argument rules): the final
 * norm + audio/text heads of the decode step, src/moss_tts/_runtime/llm.py:188-191,264-279. */
int moss_bf16_norm_gemv(const void *x, const void *res, const void *norm_w, void *sum_out, float eps, const void *w,
                        void *y, int K, int N, int rows_per_wave, void *stream);

/* ------------------------------------------------- W4A8 G32 decode mode */
/* The reference's serving arithmetic: activations quantized to int8 per group of 32, integer
 * dot products against the INT4 codes, fp32 group combine.  Quantized activations ("qact",
 * G = K/32 groups):
 *   qx    int8  [K]  in dot4 order: bytes 8b..8b+7 hold x[8b + {0,4,1,5,2,6,3,7}]
 *   sx    fp32  [G]  scale = max(RN(max|x_g| / 127), 1e-8)
 *   qsum  int32 [G]  sum of the group's codes (the zero-point term)
 * with q = rint(x * RN(1 / scale)), ties to even, |q| <= 127.
 * bf16 x [K] (K % 32 == 0) -> qact.  Replaces _int8_activation_grouped,
 * src/moss_tts/_runtime/int4_dp4a.py:21-30 (launched by dp4a_scaled.py:88-89). */
int moss_int8_quantize_g32(const void *x, void *qx, void *sx, void *qsum, int K, void *stream);

/* (add+)RMSNorm exactly as moss_rmsnorm, then the output quantized to qact (n % 32 == 0);
 * y may be NULL (no bf16 output).  For rows > 1, row r's qact starts at qx + r*n,
 * sx + r*n/32, qsum + r*n/32.  Replaces _norm_quant, src/moss_tts/_runtime/dp4a_fusions.py:24-40
 * (the normalization half of dp4a_norm_projection.py:66-78). */
int moss_rmsnorm_quant_g32(const void *x, const void *res, const void *w, void *sum_out, void *y, void *qx,
                           void *sx, void *qsum, int rows, int n, float eps, void *stream);

/* y bf16 [N] = bf16(sum_g f32(isum[n,g]) * (s[n,g] * sx[g])), isum[n,g] = sum_{k in g}
 * (q[n,k] - z[n,g]) * qx[k] exact in int32, on rowpack weights; K % 64 == 0, K <= 16384,
 * rows_per_wave in {0 (auto), 1, 2, 4}.  The fp32 sum runs over slices of 64 groups: each
 * slice's terms in a fixed tree, the slice sums in order; every W4A8 projection here uses that
 * order, so fused and unfused forms agree bit for bit.  Replaces linear (paired=False),
 * src/moss_tts/_runtime/dp4a_scaled.py:22-57,80-95 (and int4_dp4a.py:33-74). */
int moss_w4a8_gemv(const void *qx, const void *sx, const void *qsum, const void *qw, const void *sc, const void *zp,
                   void *y, int K, int N, int rows_per_wave, void *stream);

/* The same from bf16 x [K] (16-byte aligned): the int8 group quantizer runs inside the
 * projection's kernel, bit-identical to moss_int8_quantize_g32 followed by moss_w4a8_gemv.
 * Replaces linear with prequantized=None, src/moss_tts/_runtime/dp4a_scaled.py:80-95 (its
 * _int8_activation_grouped launch, :86-89, and the _gemv launch, :94). */
int moss_w4a8_quant_gemv(const void *x, const void *qw, const void *sc, const void *zp, void *y, int K, int N,
                         int rows_per_wave, void *stream);

/* Paired gate||up (W has 2*N_half rows, gate first): gate and up rounded to bf16, y bf16
 * [N_half] = bf16(bf16(silu(gate)) * up).  With out_qx/out_sx/out_qsum (all set or all NULL;
 * N_half % 32 == 0, rows_per_wave 0, 2 or 4) y is also quantized to qact for the next
 * projection.  Replaces linear
 * (paired=True, fused), src/moss_tts/_runtime/dp4a_scaled.py:60-78 (dp4a_gateup_quant.py:11-33). */
int moss_w4a8_gateup_silu(const void *qx, const void *sx, const void *qsum, const void *qw, const void *sc,
                          const void *zp, void *y, void *out_qx, void *out_sx, void *out_qsum, int K, int N_half,
                          int rows_per_wave, void *stream);

/* (add+)RMSNorm + int8 group quantizer + W4A8 projection in one kernel: x bf16 [K] (and res:
 * s = bf16(x + res), stored to sum_out, which must not overlap x or res; res and sum_out are both
 * NULL or both set), norm_w bf16 [K], K in {2048, 4096, 8192}; the
 * activations equal moss_rmsnorm_quant_g32's bit for bit, y as moss_w4a8_gemv.  Replaces the
 * fused norm + quantize + projection of src/moss_tts/_runtime/dp4a_norm_projection.py:48-166. */
int moss_w4a8_norm_gemv(const void *x, const void *res, const void *norm_w, void *sum_out, float eps, const void *qw,
                        const void *sc, const void *zp, void *y, int K, int N, int rows_per_wave, void *stream);

/* The same in front of the paired gate||up with the SiLU*mul epilogue (y bf16 [N_half], as
 * moss_w4a8_gateup_silu without output quantization).  Replaces gateup_cluster,
 * src/moss_tts/_runtime/gateup_cluster.py:44-157 (its norm + quantize + gate/up part). */
int moss_w4a8_norm_gateup_silu(const void *x, const void *res, const void *norm_w, void *sum_out, float eps,
                               const void *qw, const void *sc, const void *zp, void *y, int K, int N_half,
                               int rows_per_wave, void *stream);

/* ------------------------------------------------------------- prefill GEMM */
/* Y bf16 [M, N] = X bf16 [M, K] . dequant(W)^T with W row-packed INT4-G32 (K % 64 == 0);
 * weights are dequantized bit-exactly (bf16_rne((q-z)*s)), in the registers that feed
 * v_mfma_f32_32x32x16_bf16 (M > 64) or into LDS, fp32 accumulate.  2 to 4 tokens (4 only for
 * K <= 4096) take the multi-token GEMV of moss_w4g32_gemv instead (no matrix cores; each row of Y
 * equal to the single-token GEMV's).  When the output tiles alone
 * cannot fill the GPU the K dimension is split over workgroups: that needs a caller-owned fp32 workspace
 * of moss_gemm_workspace_bytes(M, K, N) bytes (16-byte aligned; y 8-byte aligned); with a
 * NULL or smaller workspace the GEMM runs unsplit.  Partial sums are added in a fixed order.
 * The reference runs bf16 F.linear here (src/moss_tts/_runtime/llm.py:29,84,130); its INT4
 * contract is dequant + F.linear (src/moss_tts/calibration.py:185-188). */
int moss_w4g32_gemm(const void *x, const void *qw, const void *sc, const void *zp, void *y, int M, int K, int N,
                    void *workspace, long long workspace_bytes, void *stream);

/* Workspace bytes the GEMMs (INT4 and FP8, M > 1) use for an M x K x N problem; 0 = none. */
long long moss_gemm_workspace_bytes(int M, int K, int N);

/* Prefill gate||up projection with the SiLU*mul epilogue: qw/sc/zp hold 2*N rows (gate rows, then
 * up rows; N % 4 == 0), y bf16 [M, N] = bf16(bf16(silu(g)) * u) with g, u the bf16 outputs of
 * moss_w4g32_gemm on those rows -- equal bit for bit to moss_w4g32_gemm (full workspace) followed by
 * moss_silu_mul.  For M > 64 where the GEMM plan has no K split (Qwen3-8B's gate||up at every
 * M > 64) the epilogue runs inside the GEMM and no [M, 2N] product is written; otherwise the
 * product and the GEMM's partial sums go to a caller-owned workspace of
 * moss_gemm_silu_workspace_bytes(M, K, N) bytes (16-byte aligned; for 16/8-byte aligned sc/zp and
 * 8-byte aligned y -- otherwise the unfused form runs and needs that workspace too, and a smaller
 * one is refused with hipErrorInvalidValue).  Replaces F.linear(x, _gate_up) followed by the
 * prefill SiLU (src/moss_tts/_runtime/llm.py:27-29, prefill_pointwise.py:18-31). */
int moss_w4g32_gemm_silu(const void *x, const void *qw, const void *sc, const void *zp, void *y, int M, int K, int N,
                         void *workspace, long long workspace_bytes, void *stream);

/* Workspace bytes that always suffice for moss_w4g32_gemm_silu on an M x K x N problem (N = the SiLU
 * outputs): the unfused form's, since whether the fused tile runs also depends on the pointers'
 * alignment, which this query does not see. */
long long moss_gemm_silu_workspace_bytes(int M, int K, int N);

/* Prefill QKV projection (N = 6144: 32 query, 8 key, 8 value heads of 128) with the q/k head
 * RMSNorm + RoPE and the K/V cache write as its epilogue: equal bit for bit to moss_w4g32_gemm
 * (full workspace) followed by moss_qk_norm_rope_kv(..., cos_by_position = 1).  q_out bf16
 * [M, 32, 128]; K/V rows positions[t] (int64 [M], clamped into 0 .. L - 1) of the [8, L, 128]
 * caches; cos/sin [L, 128]; q_weight/k_weight [128].  For M > 64 where the GEMM plan has no K split
 * (Qwen3-8B at M > 256) the norm, RoPE and cache writes run inside the GEMM and no [M, 6144]
 * product is written; otherwise the GEMM's output goes to a caller-owned workspace of
 * moss_gemm_qk_rope_workspace_bytes(M, K) bytes (16-byte aligned; also for sc/zp not 16/8-byte
 * aligned), and a K-split plan's fp32 partials are reduced by the RoPE kernel itself, in split
 * order.  x, qw 16-byte aligned; the bf16 vectors, caches, q_out and positions
 * 8-byte aligned.  Replaces qkv_proj and the prefill q/k-norm + RoPE + cache write
 * (src/moss_tts/_runtime/llm.py:84, :95-98, prefill_qkv.py:31-53). */
int moss_w4g32_gemm_qk_rope(const void *x, const void *qw, const void *sc, const void *zp, const void *q_weight,
                            const void *k_weight, const void *cos, const void *sin, void *q_out, void *k_cache,
                            void *v_cache, const void *positions, int M, int K, int L, float eps, void *workspace,
                            long long workspace_bytes, void *stream);

/* Workspace bytes that always suffice for moss_w4g32_gemm_qk_rope on M tokens of K inputs (the
 * unfused form's, as for moss_gemm_silu_workspace_bytes). */
long long moss_gemm_qk_rope_workspace_bytes(int M, int K);

/* Prefill O / down projection followed by the residual add and RMSNorm: with p = the bf16 product
 * of moss_w4g32_gemm, summed_out = bf16(p + residual) and y = bf16(bf16(summed * rsqrt(mean(summed^2)
 * + eps)) * norm_w), both [M, N] (N % 8 == 0, N <= 8192; x, residual, norm_w, summed_out, y 16-byte
 * aligned) -- equal bit for bit to moss_w4g32_gemm followed by moss_rmsnorm with the residual.  The
 * workspace is moss_w4g32_gemm's (moss_gemm_workspace_bytes); when the plan splits K, the norm
 * kernel reduces the partial sums itself (one launch and one [M, N] round trip fewer).  summed_out
 * and y must not overlap x, residual or each other (an in-place residual update is refused with
 * hipErrorInvalidValue).  Replaces o_proj / down_proj and the following add_rmsnorm of the prefill
 * layer loop (src/moss_tts/_runtime/llm.py:84, prefill_pointwise.py:46-57). */
int moss_w4g32_gemm_add_rmsnorm(const void *x, const void *qw, const void *sc, const void *zp, const void *residual,
                                const void *norm_w, float eps, void *summed_out, void *y, int M, int K, int N,
                                void *workspace, long long workspace_bytes, void *stream);

/* moss_w4g32_gemm without a workspace argument and without any allocation: the K-split partial sums
 * go to a 32 MiB device array inside the library (one per GPU, kept until the process ends), which
 * holds every plan's partials, so the result equals moss_w4g32_gemm's with a full workspace bit for
 * bit.  A shape whose plan would need more is refused with hipErrorInvalidValue.  The array's device
 * address is looked up on the first call on each device (make that call outside graph capture);
 * calls that overlap on one device share the array and race.  No counterpart in the reference: for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int moss_w4g32_gemm_noalloc(const void *x, const void *qw, const void *sc, const void *zp, void *y, int M, int K,
                            int N, void *stream);

/* --------------------------------------------------- FP8 E4M3 weight-only */
/* W e4m3 (OCP) [N, K] row-major bytes (16-byte aligned), scale fp32 [N] or NULL (= 1):
 * y bf16 [M, N] = bf16(scale[n] * sum_k f32(W[n,k]) * x[m,k]), fp32 accumulate.
 * M == 1: decode GEMV (K % 16 == 0, K <= 16384, rows_per_wave in {0 (auto), 1, 2, 4});
 * M > 1: MFMA GEMM with exact e4m3 -> bf16 weights (K % 64 == 0), optionally split over K
 * with the workspace described at moss_w4g32_gemm.  Arithmetic of _fp8_silu_gemv,
 * src/moss_tts/_runtime/fused_mlp.py:7-23, without the SiLU epilogue. */
int moss_fp8_linear(const void *x, const void *w, const void *scale, void *y, int M, int K, int N,
                    int rows_per_wave, void *workspace, long long workspace_bytes, void *stream);

/* Fused gate||up FP8 decode GEMV: W e4m3 [2*N_half, K] (gate rows first), scale fp32
 * [2*N_half] or NULL, M must be 1; y bf16 [N_half] = bf16(bf16(silu(bf16(g*sg))) *
 * bf16(u*su)).  Replaces fp8_silu_decode, src/moss_tts/_runtime/fused_mlp.py:26-30. */
int moss_fp8_gateup_silu(const void *x, const void *w, const void *scale, void *y, int M, int K, int N_half,
                         int rows_per_wave, void *stream);

/* e4m3 [count] -> bf16 [count] (count % 4 == 0), exact.  The weight conversion the FP8
 * kernels apply, exposed for checking (torch's float8_e4m3fn -> bfloat16 cast). */
int moss_fp8_to_bf16(const void *w, void *out, long long count, void *stream);

/* --------------------------------------------------- norms, RoPE, SiLU*mul */
/* Row RMSNorm over n (n % 8 == 0, n <= 8192), bf16 in/out, rounding points of Qwen3RMSNorm.
 * res == NULL: y = rmsnorm(x) (src/moss_tts/_runtime/kernels.py:50-66).
 * res != NULL: sum_out = bf16(x + res); y = rmsnorm(sum_out) (kernels.py:69-90). */
int moss_rmsnorm(const void *x, const void *res, const void *w, void *sum_out, void *y, int rows, int n, float eps,
                 void *stream);

/* Qwen3-8B q/k head RMSNorm + RoPE + KV-cache write for ntok tokens.
 * qkv bf16 [ntok, 6144] (q 32x128 | k 8x128 | v 8x128), q/k norm weights bf16 [128],
 * cos/sin bf16 rows of 128: row t of [ntok, 128] (cos_by_position = 0) or row positions[t]
 * of a [L, 128] table (cos_by_position = 1, so a captured decode graph stays valid for any
 * position), positions int64 [ntok] (unique, in [0, L); clamped), q_out bf16 [ntok, 32, 128],
 * caches bf16 [8, L, 128] written at rows positions[t].
 * Replaces _qk_rope_cache (src/moss_tts/_runtime/kernels.py:142-170) and _prefill_qkv
 * (src/moss_tts/_runtime/prefill_qkv.py:7-28, project :61-83). */
int moss_qk_norm_rope_kv(const void *qkv, const void *q_weight, const void *k_weight, const void *cos,
                         const void *sin, void *q_out, void *k_cache, void *v_cache, const void *positions, int L,
                         int ntok, float eps, int cos_by_position, void *stream);

/* x bf16 [rows, 2n] = (gate | up) halves of width n (n even) -> y bf16 [rows, n],
 * y = bf16(bf16(silu(g)) * u).  Replaces _silu mode 0 of
 * src/moss_tts/_runtime/prefill_pointwise.py:18-31 and _silu_mul, kernels.py:123-139. */
int moss_silu_mul(const void *x, void *y, int rows, int n, void *stream);

/* ------------------------------------------------------- decode attention */
/* Number of 64-row splits for a cache of L rows (sizes partial [32, S, 128] fp32, lse [32, S]). */
int moss_decode_attention_splits(int L);

/* One query token, Qwen3-8B GQA (32 query / 8 KV heads, head_dim 128): q bf16 [32,128],
 * caches bf16 [8, L, 128] (one layer of the [1, 8, L, 128] static cache, L % 64 == 0,
 * L <= 32768), position int64 [1] on the device (rows 0..position are attended; clamped to
 * L-1), caller-owned workspace partial fp32 [32, S, 128] and lse fp32 [32, S] (S = L / 64;
 * calls sharing a workspace must not overlap), out bf16 [32 * 128].  Two launches: 64-row
 * splits, then a log-sum-exp merge in split order.
 * Replaces _decode_attn/_decode_attn_reduce (src/moss_tts/_runtime/kernels.py:173-208,
 * driven from qk_rope_decode :211-251) and launch_attention_ordered
 * (src/moss_tts/_runtime/attention_native.cu:91-97). */
int moss_decode_attention(const void *q, const void *k_cache, const void *v_cache, const void *position,
                          void *partial, void *lse, void *out, int L, void *stream);

/* q/k head-norm + RoPE + KV-cache write + decode attention in one pass: qkv bf16 [6144]
 * (q 32x128 | k 8x128 | v 8x128, raw projection output), q/k head-norm weights bf16 [128],
 * cos/sin bf16 [L, 128] tables (row = position), the rest as moss_decode_attention.  Row
 * `position` of both caches is written (by the one split that holds it, which also uses the new
 * row directly).  Bit-identical to moss_qk_norm_rope_kv (ntok 1, cos_by_position 1) followed by
 * moss_decode_attention.  Replaces qk_rope_decode, src/moss_tts/_runtime/kernels.py:211-251. */
int moss_decode_attention_qkv(const void *qkv, const void *q_norm_w, const void *k_norm_w, const void *cos_t,
                              const void *sin_t, void *k_cache, void *v_cache, const void *position, void *partial,
                              void *lse, void *out, int L, float eps, void *stream);

/* moss_decode_attention_qkv whose merge also quantizes its bf16 output for the W4A8 O projection:
 * out_qx int8 [4096] in dot4 order, out_sx fp32 [128] and out_qsum int32 [128] per group of 32, as
 * moss_int8_quantize_g32 forms them from out.  Replaces reduce_quant,
 * src/moss_tts/_runtime/attention_quant.py:8-32. */
int moss_decode_attention_qkv_quant(const void *qkv, const void *q_norm_w, const void *k_norm_w, const void *cos_t,
                                    const void *sin_t, void *k_cache, void *v_cache, const void *position,
                                    void *partial, void *lse, void *out, void *out_qx, void *out_sx, void *out_qsum,
                                    int L, float eps, void *stream);

/* Causal GQA attention of the prompt pass (Qwen3-8B: 32 query / 8 KV heads, head_dim 128):
 * q bf16 [n, 32, 128] for the tokens at absolute positions *start .. *start + n - 1 (start int64 [1]
 * on the device, clamped to [0, L - n]), whose K/V rows are already in the caches bf16 [8, L, 128]
 * (L % 64 == 0, n <= L <= 32768); token t attends rows 0 .. *start + t with scale 1/sqrt(128),
 * softmax in fp32, probabilities rounded to bf16 for the P.V product; out bf16 [n, 32 * 128].
 * Replaces F.scaled_dot_product_attention(..., is_causal=True, enable_gqa=True) of the prefill
 * forward, src/moss_tts/_runtime/llm.py:116-128. */
int moss_prefill_attention(const void *q, const void *k_cache, const void *v_cache, const void *start, void *out,
                           int n, int L, void *stream);

/* ids int64 [T, Q+1] (text token then Q codebook codes), text bf16 [Vt, H], audio bf16
 * [Q, V, H] -> out bf16 [T, H] with a bf16 rounding after each addition; ids are clamped
 * into their tables.  Replaces embedding_sum (src/moss_tts/_runtime/kernels.py:7-26). */
int moss_embedding_sum(const void *ids, const void *text, const void *audio, void *out, int T, int H, int Vt, int V,
                       int Q, void *stream);

/* --------------------------------------------------------------- sampling */
/* Per row of bf16 logits (rows x stride, the first `vocab` <= 2048 entries used): temperature <= 0
 * gives the argmax (first maximal index); otherwise the top_k (1..64) largest of logits/temperature
 * in fp32, descending (ties: lower index first), their softmax, entries whose preceding cumulative
 * probability exceeds top_p removed, and one index drawn in proportion to the rest with a Philox4x32-10
 * uniform (counter = (*position, row, salt), key = *seed).  seed uint64 [1] and position int64 [1] are
 * device buffers read when the kernel runs, so a captured graph follows new seeds and positions.
 * out int64 [rows].
 * Replaces sample_topk, src/moss_tts/_runtime/llm.py:10-19 (torch.topk + softmax + multinomial). */
int moss_sample_topk(const void *logits, int rows, int stride, int vocab, float temperature, int top_k, float top_p,
                     const void *seed, const void *position, int salt, void *out, void *stream);

/* Two moss_sample_topk calls with one seed and position in one launch (the decode step's text row
 * and its audio rows): set a's rows_a rows, then set b's rows_b rows, each row sampled exactly as
 * moss_sample_topk samples it (row numbers restart at 0 in set b), so the outputs equal the two
 * separate calls'.  Replaces the pair of sample_topk calls of src/moss_tts/_runtime/llm.py:280,284. */
int moss_sample_topk_pair(const void *logits_a, int rows_a, int stride_a, int vocab_a, float temperature_a,
                          int top_k_a, float top_p_a, int salt_a, void *out_a, const void *logits_b, int rows_b,
                          int stride_b, int vocab_b, float temperature_b, int top_k_b, float top_p_b, int salt_b,
                          void *out_b, const void *seed, const void *position, void *stream);

/* next_ids int64 [1 + channels] from the sampled text index (int64 [1], into text_ids int64 [2]) and
 * audio indices (int64 [channels]): the text token becomes delay_slot_id while *delay_length >= 0 and
 * audio_end_id at *delay_length == 32; audio code c is kept when c < *audio_length and
 * (*delay_length < 0 or c >= *delay_length), else pad_code.  Replaces the token logic of _decode,
 * src/moss_tts/_runtime/llm.py:280-287. */
int moss_compose_next_ids(const void *text_index, const void *audio_index, const void *text_ids,
                          const void *audio_length, const void *delay_length, long long delay_slot_id,
                          long long audio_end_id, int channels, long long pad_code, void *next_ids, void *stream);

/* One in-audio step of the host loop on the device, so several decode steps can run in one graph:
 * ids int64 [width] <- next_ids [width] (and history[step * width ...] when history is not null);
 * *position += 1; *audio_length += 1 when next_ids[0] is audio_start_id, gen_slot_id or delay_slot_id;
 * *delay_length becomes 0 at the first delay_slot_id and then grows by 1 each step; status int64 [4]
 * (optional) = (text token, audio length, delay, position) after the update.  next_ids != ids.
 * Replaces the host update of src/moss_tts/_runtime/streaming.py:107-112 and the _advance kernel of
 * src/moss_tts/_runtime/first_audio_graph.py:14-29. */
int moss_advance_step(const void *next_ids, void *ids, void *position, void *audio_length, void *delay_length,
                      void *history, void *status, int step, int width, long long audio_start_id,
                      long long gen_slot_id, long long delay_slot_id, void *stream);

/* ------------------------------------------------------- measurement */
/* No counterpart in the reference: a streaming read for bench.py, which times it on the bytes of a
 * decode GEMV to measure the ceiling of one launch that only reads those bytes.  Reads `bytes` (a
 * multiple of 16) from the 16-byte aligned src with 16-byte loads, one 256-thread workgroup per
 * 16 KiB (thread t of workgroup b reads chunks 1024 b + 256 u + t, u < 4), and writes the XOR of
 * the 32-bit words each wave read to xor_out[4 b + t / 64] (uint32, moss_stream_read_words(bytes)
 * entries). */
long long moss_stream_read_words(long long bytes);
int moss_stream_read(const void *src, long long bytes, void *xor_out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MOSS_HIP_H */
