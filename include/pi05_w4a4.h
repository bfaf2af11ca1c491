/*
 * pi05_w4a4.h -- C ABI of the MI355X (gfx950) W4A4 prefix-LM GEMM library
 * (libpi05_w4a4.so, built by hipcc --offload-arch=gfx950).
 *
 * The library replaces the pybind module that the reference JIT-builds from
 * pi05_fast/w4a4/csrc/int4_gemm.cu (PYBIND11_MODULE at int4_gemm.cu:644-650).  The
 * host mirror of the reference's op surface (pi05_fast.w4a4.extension) binds these
 * symbols through ctypes.  Signatures carry plain device pointers, sizes and a HIP
 * stream (as void*), never torch types.  The library allocates no device memory:
 * outputs, quantized activations and workspaces are allocated by the caller.
 *
 * Every entry point returns a status code (PI05W4A4_OK on success).  A non-zero code
 * comes with a message retrievable through pi05w4a4_last_error() (thread-local).
 * Kernels are launched asynchronously on `stream`; nothing synchronises the host.
 *
 * Data formats
 *   x      fp16 [M, K] row-major activations (K % 64 == 0), 16-byte aligned.
 *   q      nibble-packed activation codes (values in [-7, 7]) in the MFMA-fragment-major
 *          layout shared with the weights.  Byte j of a word holds the codes of k = 2j
 *          (low nibble, offset binary: code + 8) and k = 2j + 1 (high nibble, two's
 *          complement); the reference's word is this word XOR 0x08080808.
 *          With KB = ceil(K/128),
 *          the codes of 16-row block mb and 128-deep k block b form one 1 KB fragment at
 *          word (mb*KB + b)*256 made of 64 16-byte slots: slot L (words 4L .. 4L+3) holds
 *          codes 128*b + 32*(L/16) .. +31 of row 16*mb + L%16, code k in nibble (k & 7)
 *          of its word (encoded as above).  Lane L of an MFMA wave loads slot L and feeds its codes 0-15 and
 *          16-31 to the block's two v_mfma_i32_16x16x64_i8.  Row-major word (row, kw) of
 *          the reference's [M, K/8] codes therefore sits at
 *          ((row/16)*KB + kw/16)*256 + 4*(row%16 + 16*((kw%16)/4)) + kw%4.
 *          The codes of ceil(M/16)*16 rows (K rounded up to 128) are followed by one
 *          int32 per row, qcorr[row] = -128 * (sum of the row's odd-k codes): the GEMM
 *          unpacks each code byte with one AND and needs these to undo the offsets.
 *          The buffer holds pi05w4a4_q_words(M, K) words (padding is never read into
 *          an output).  16-byte aligned.
 *   sa     fp32 [M] per-token activation scales.
 *   w_mfma weights in the gfx950 MFMA-fragment-major layout (see
 *          pi05w4a4_repack_weight).  N % 16 == 0.  Word count pi05w4a4_mfma_words().
 *          16-byte aligned.
 *   y      fp16 [M, N] row-major outputs, 16-byte aligned.
 */
#ifndef PI05_W4A4_H_
#define PI05_W4A4_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PI05W4A4_OK 0
#define PI05W4A4_EINVAL 1     /* invalid argument (shape, alignment, null pointer) */
#define PI05W4A4_EHIP 2       /* HIP runtime / launch error */
#define PI05W4A4_EWORKSPACE 3 /* workspace too small */

/* Source layouts accepted by pi05w4a4_repack_weight. */
#define PI05W4A4_LAYOUT_ROW_MAJOR 0 /* L1 [N, K/8+1] / L2 [N, K/8+P]: row stride = src_stride */
#define PI05W4A4_LAYOUT_WMMA_TILED 1 /* L3 [N, K/8+9] read flat: flat[(t*N+n)*2+h] = L1[n,2t+h] */

/* Extra words per row of the persistent MFMA tensor [N, K/8 + 16] ("MFMA marker stride"). */
#define PI05W4A4_MFMA_MARKER_WORDS 16

/* Library version (major*10000 + minor*100 + patch). */
int pi05w4a4_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* pi05w4a4_last_error(void);

/*
 * Fused Walsh-Hadamard rotation + per-token symmetric INT4 quantization + nibble pack.
 * Replaces quantize_x / quant_rot_rb / quant_rows (int4_gemm.cu:396-477, 496-531).
 * Rotation iff K in {1024, 2048, 16384} (unnormalised Sylvester FWHT, staged in fp32);
 * sdiv = amax/7 + 1e-12; q = clamp(rint(x'/sdiv), -7, 7);
 * sa = sdiv * fp32(1/sqrt(K)) when rotated, else sdiv.
 */
int pi05w4a4_quantize(const void* x_fp16, int64_t m, int32_t k, int32_t* q, float* sa,
                      void* stream);

/*
 * pi05w4a4_quantize plus cache warming: at K = 16384 (one 68 KB workgroup per row, two per
 * CU) the workgroup slots that the last round of rows leaves idle read warm_n <= 4 further
 * device buffers (16-byte aligned, sizes multiples of 16 bytes) and discard the data, so
 * that the kernels after it find them in the Infinity Cache; other K ignore the buffers.
 * No counterpart in the reference: the fused decoder layer passes the down-proj weights
 * with the quantization of the down-proj input.  Results are those of pi05w4a4_quantize.
 */
int pi05w4a4_quantize_warm(const void* x_fp16, int64_t m, int32_t k, int32_t* q, float* sa,
                           const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                           void* stream);

/*
 * Words of a quantized-activation buffer q for M rows of K codes:
 * ceil(M/16)*16 * ceil(K/128)*16 code words + ceil(M/16)*16 qcorr words.
 * (The reference keeps row-major [M, K/8] codes inside its QuantizedX, int4_gemm.cu:479-485.)
 */
size_t pi05w4a4_q_words(int64_t m, int32_t k);

/*
 * Words of the MFMA-fragment-major weight buffer for an [N, K] weight: payload
 * N*ceil(K/128)*16 words, then N fp32 scale words, then N wcorr words.  The persistent tensor form is
 * int32 [N, K/8 + PI05W4A4_MFMA_MARKER_WORDS], which always holds that many words.
 */
size_t pi05w4a4_mfma_words(int32_t n, int32_t k);

/*
 * One-time weight repack into the MFMA-fragment-major layout.
 * Replaces the reference's load-time layout handling: row padding (apply.py:68-69),
 * preshuffle_wmma_weight (pack.py:45-68) and the kernel-side addressing
 * weight_word_offset / weight_scale_offset (int4_gemm.cu:44-61).
 *   src        device int32 weights in `src_layout`;
 *   src_stride row stride in words for PI05W4A4_LAYOUT_ROW_MAJOR (>= K/8 + 1), ignored
 *              for PI05W4A4_LAYOUT_WMMA_TILED;
 *   dst        device buffer of at least pi05w4a4_mfma_words(n, k) int32 words.
 * Layout of dst: the q layout above applied to weight columns (column n in place of row
 * `row`) with the weight nibble encoding: byte j holds the code of k = 2j in its high
 * nibble (two's complement) and that of k = 2j + 1 in its low nibble (offset binary).
 * K is padded to a multiple of 128 with zero words.  Then dst[P + n] = scale bits of
 * column n and dst[P + N + n] = wcorr[n] = -128 * (sum of column n's even-k codes),
 * P = N*ceil(K/128)*16.
 */
int pi05w4a4_repack_weight(const int32_t* src, int32_t src_layout, int32_t n, int32_t k,
                           int64_t src_stride, int32_t* dst, void* stream);

/*
 * Exact workspace bytes that pi05w4a4_gemm / _gemm_multi (gelu = 0) or
 * pi05w4a4_gemm_gelu_up (gelu = 1, ngroups = 2, n = {N, N}) need for an (M, K)
 * activation against weights of n[0..ngroups-1] columns.  0 means no workspace.
 * The workspace holds split-K int32 partial sums; it is fully overwritten by each call
 * (no zeroing needed), so calls that share one workspace must be stream-ordered.
 */
size_t pi05w4a4_gemm_workspace_bytes(int64_t m, int32_t k, int32_t ngroups, const int32_t* n,
                                     int32_t gelu);

/*
 * y = fp16((float(acc) * sa[m]) * sw[n]), acc[m,n] = sum_k q[m,k] * w[n,k] in int32.
 * Replaces gemm_from_q + gemm_iu4 / gemm_iu4_shape (int4_gemm.cu:63-394, 566-616).
 * All GEMM entry points accept K up to 524288 (the int32 MFMA sum is at most 2048 K).
 */
int pi05w4a4_gemm(const int32_t* q, const float* sa, int64_t m, int32_t k,
                  const int32_t* w_mfma, int32_t n, void* y_fp16, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * Shared-activation GEMM against 1..3 weights of equal K in one launch
 * (the fan-out of int4_gemm2 / int4_gemm3, int4_gemm.cu:626-642).
 * w_mfma[g], n[g], y_fp16[g] for g < ngroups.
 */
int pi05w4a4_gemm_multi(const int32_t* q, const float* sa, int64_t m, int32_t k,
                        int32_t ngroups, const int32_t* const* w_mfma, const int32_t* n,
                        void* const* y_fp16, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * Fused gate/up GEMM with a GELU-tanh(gate) * up epilogue: h = fp16(gelu_tanh(g) * u)
 * where g, u are the fp16-rounded gate/up outputs.  Replaces the int4_gemm2 call plus
 * the elementwise `act_fn(gate) * up` of apply.py:135-138 (one rounding fewer).
 */
int pi05w4a4_gemm_gelu_up(const int32_t* q, const float* sa, int64_t m, int32_t k,
                          const int32_t* w_gate_mfma, const int32_t* w_up_mfma, int32_t n,
                          void* h_fp16, void* workspace, size_t workspace_bytes, void* stream);

/*
 * pi05w4a4_gemm_gelu_up followed by the down projection's activation quant of its output:
 * h as above, then dq / dsa = pi05w4a4_quantize(h, M, K = n) (codes, row corrections and
 * scales bit for bit; dq holds pi05w4a4_q_words(M, n) words).  Replaces the MLP's
 * `act_fn(gate) * up` followed by the down projection's quantize_x (apply.py:135-141,
 * int4_gemm.cu:496-531).  At n = 16384 with M > 64 both run in one launch: workgroups
 * appended to the GEMM tiles quantize each 112-row block of h as soon as all of its
 * columns are stored, in the slots the GEMM's partial last round leaves idle (other
 * shapes: two launches, same results).
 * ctl: int32 control block of pi05w4a4_mlp_ctl_words(M) words in device memory, zeroed
 * once by the caller before its first use; every call that completes leaves it zeroed.
 * Calls that share one control block must be stream-ordered (calls that overlap race).
 * warm_*: up to 4 buffers read into the Infinity Cache by quant workgroups that find no
 * row left (pi05w4a4_quantize_warm's argument form).
 * The quant workgroups wait for the GEMM tiles of their row block with a bounded wait
 * (spin_limit rounds of about 4 us; 0 = the default of 2^20) that never deadlocks (see
 * the kernel); one that runs out leaves its row unquantized and sets a host-visible status
 * word, read by pi05w4a4_mlp_status: the outputs of that call are invalid and ctl must be
 * zeroed again.  wait_extra (0 in normal use; tests pass 1) makes every wait expect one
 * completion more than exists, which forces that path.
 * No counterpart in the reference (an optional fusion of two of its steps).
 */
int pi05w4a4_gemm_gelu_up_quant(const int32_t* q, const float* sa, int64_t m, int32_t k,
                                const int32_t* w_gate_mfma, const int32_t* w_up_mfma, int32_t n,
                                void* h_fp16, int32_t* dq, float* dsa, int32_t* ctl,
                                const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                                int32_t spin_limit, int32_t wait_extra, void* stream);

/* Words of the control block of pi05w4a4_gemm_gelu_up_quant for M rows (0 for M <= 0). */
size_t pi05w4a4_mlp_ctl_words(int64_t m);

/*
 * Number of bounded waits of pi05w4a4_gemm_gelu_up_quant that ran out since the last
 * clear (a pinned host word the kernels write; reading it does not synchronize, so it
 * covers the calls that have completed).  clear != 0 resets it.  -1 when the word cannot
 * be allocated (no device).  No counterpart in the reference.
 */
int64_t pi05w4a4_mlp_status(int32_t clear);

/*
 * GEMM with a residual add in the epilogue: y = fp16(fp16((acc * sa[m]) * sw[n]) + r[m, n])
 * for residual r fp16 [M, N] (16-byte aligned; y may alias r).  The second rounding is
 * that of the decoder's fp16 `residual + hidden_states` (modeling_gemma.py
 * GemmaDecoderLayer.forward), which it replaces for o_proj and down_proj: the reference
 * runs int4_gemm (int4_gemm.cu:618-624) and then the add as a separate elementwise op.
 */
int pi05w4a4_gemm_residual(const int32_t* q, const float* sa, int64_t m, int32_t k,
                           const int32_t* w_mfma, int32_t n, const void* residual_fp16,
                           void* y_fp16, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Small-M quant + GEMM in one launch (1 <= M <= 4, K = 2048): the y[g] of
 * pi05w4a4_gemm_multi (or, with a residual and one weight, of pi05w4a4_gemm_residual)
 * applied to the codes and scales of pi05w4a4_quantize(x), or of
 * pi05w4a4_rmsnorm_quantize(x, nw, eps, unit_offset) when nw is not null, bit for bit.
 * Every workgroup (16 x 32 tiles whose four waves split K) quantizes the rows itself into
 * LDS while its first weight fragments load, so no activation codes are stored and the
 * separate quant launch of decode-sized calls is gone.  Replaces the reference's quantize_x
 * followed by gemm_from_q (int4_gemm.cu:496-531, 566-616) at those sizes, with the norm of
 * the following entry point when nw is given.  x, nw, the weights, y and the residual are
 * 16-byte aligned; the weights are MFMA-layout with N % 16 == 0.
 */
int pi05w4a4_quant_gemm_small(const void* x_fp16, const void* nw_fp16, float eps, int32_t unit_offset, int64_t m,
                              int32_t k, int32_t ngroups, const int32_t* const* w_mfma, const int32_t* n,
                              void* const* y_fp16, const void* residual_fp16, void* stream);

/*
 * RMSNorm fused into the K = 2048 activation quant: the codes and scales of
 * pi05w4a4_quantize applied to h = fp16((x * r) * (unit_offset + w)),
 * r = 1 / sqrt(sum(x^2) / K + eps), the input norm of every attention and MLP block of
 * the prefix LM.  Replaces the reference's GemmaRMSNorm (modeling_gemma.py:64-78) plus the
 * quantize_x of the following int4_gemm3 / int4_gemm2 (int4_gemm.cu:496-531).  The fp32
 * sum of squares runs per lane over 32 consecutive elements (lane l: elements 32l ..
 * 32l + 31, in order), then across the 64 lanes by the xor butterfly 32, 16, .., 1; sqrt
 * and the division are correctly rounded.  h differs from the eager module's output by at
 * most one fp16 ulp on a few elements (torch sums in another order and uses rsqrt).
 */
int pi05w4a4_rmsnorm_quantize(const void* x_fp16, const void* w_fp16, float eps,
                              int32_t unit_offset, int64_t m, int32_t k, int32_t* q, float* sa,
                              void* stream);

/*
 * pi05w4a4_rmsnorm_quantize plus cache warming: when the row workgroups (4 rows each) leave
 * CUs without one, a workgroup per such CU reads warm_n <= 4 further device buffers
 * (16-byte aligned, sizes multiples of 16 bytes) and discards the data, so that the GEMM
 * after it finds them in the Infinity Cache.  No counterpart in the reference: the QKV
 * entry ops pass their own weights with the quantization of their input.  Results are
 * those of pi05w4a4_rmsnorm_quantize.
 */
int pi05w4a4_rmsnorm_quantize_warm(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                   int64_t m, int32_t k, int32_t* q, float* sa, const void* const* warm_ptrs,
                                   const size_t* warm_bytes, int32_t warm_n, void* stream);

/*
 * Raw int32 accumulators acc[m, n] (row-major [M, N]) for bit-exact checks; no dequant.
 * Debug counterpart of the int32 accumulation inside gemm_iu4 (int4_gemm.cu:114-178).
 */
int pi05w4a4_gemm_acc(const int32_t* q, int64_t m, int32_t k, const int32_t* w_mfma,
                      int32_t n, int32_t* acc, void* stream);

/*
 * Convenience: quantize + GEMM(s), mirroring the reference's host entry points
 * int4_gemm / int4_gemm2 / int4_gemm3 (int4_gemm.cu:618-642) for MFMA-layout weights.
 * `qbuf` must hold pi05w4a4_q_words(M, K) int32 words and `sabuf` M floats.
 */
int pi05w4a4_int4_gemm(const void* x_fp16, int64_t m, int32_t k, const int32_t* w_mfma,
                       int32_t n, void* y_fp16, int32_t* qbuf, float* sabuf, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * Allocation-free pi05w4a4_int4_gemm: quantize + GEMM of one MFMA-layout weight with the
 * activation codes, row scales and split-K partials in a fixed device scratch array that
 * the library holds on each GPU it runs on (PI05W4A4_NOALLOC_SCRATCH_BYTES, kept until the
 * process ends) instead of caller buffers.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc); it calls no allocating routine.  Same
 * arguments, checks and results as pi05w4a4_int4_gemm without qbuf / sabuf / workspace;
 * a call whose buffers would exceed the scratch size fails with PI05W4A4_EINVAL before
 * any launch.  Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * device (other streams, other host threads) race and must be serialised by the caller.
 * Footprint: the scratch is a static device array of the library, so every GPU that the
 * library is loaded on reserves these 64 MiB of HBM until the process ends, whether or not
 * this entry point is called.
 */
#define PI05W4A4_NOALLOC_SCRATCH_BYTES (64u << 20)
int pi05w4a4_int4_gemm_noalloc(const void* x_fp16, int64_t m, int32_t k, const int32_t* w_mfma,
                               int32_t n, void* y_fp16, void* stream);

/*
 * Elementwise y = fp16(gelu_tanh(gate) * up) on fp16 [n] arrays (y may alias either input),
 * with the arithmetic of pi05w4a4_gemm_gelu_up's epilogue.  Replaces the eager
 * `gelu(gate, approximate="tanh") * up` of the unfused MLP (apply.py:135-138); the result
 * equals those two eager fp16 ops bit for bit.
 */
int pi05w4a4_gelu_tanh_mul(const void* gate_fp16, const void* up_fp16, int64_t n, void* y_fp16,
                           void* stream);

/*
 * RMSNorm of fp16 rows, the input norm of every attention and MLP block ahead of the QKV
 * and gate/up activation quant.  No counterpart in the reference's W4A4 code: it replaces
 * transformers' GemmaRMSNorm module (modeling_gemma.py:64-78), which the reference runs
 * eagerly between its W4A4 ops, with one kernel of the same fp32 operations:
 *   y = fp16((float(x) * r) * (unit_offset + float(w))),
 *   r = 1 / sqrt(sum(float(x)^2) * fp32(1/K) + eps)   (correctly rounded sqrt and division).
 * x, y fp16 [M, K] (may alias), w fp16 [K]; K % 8 == 0, K <= 16384; 16-byte aligned.
 * The sum of squares has the fixed lane order of pi05w4a4_rmsnorm_quantize's norm, so both
 * entry points produce the same fp16 rows; torch sums in another order and rounds its
 * rsqrt differently, so a few outputs can differ from the eager module's by one fp16 ulp.
 */
int pi05w4a4_rmsnorm(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                     int64_t m, int32_t k, void* y_fp16, void* stream);

/*
 * Prefix attention between the QKV and o projections, head_dim 256, H query heads sharing
 * KVH key/value heads, fp16.  No counterpart in the reference's W4A4 code: it replaces
 * the RoPE and eager attention that the reference's fused attention forward runs between
 * int4_gemm3 and o_proj (apply.py:167-188: transformers' apply_rotary_pos_emb and
 * eager_attention_forward) with two kernels of the same fp16/fp32 operation order:
 *   q', k' = fp16(fp16(x * cos) + fp16(rotate_half(x) * sin))          (bit-exact)
 *   s = fp16(fp16(fp16(q' . k') * scaling) + mask); p = fp16(softmax_fp32(s)); o = fp16(p v)
 * The fp32 sums run in another order than torch's and exp uses the hardware exp2, so o
 * agrees with the eager output to fp16 rounding.  S (keys = queries) is at most 1024.
 *
 * pi05w4a4_attn_kv_prep: k, v fp16 [B, S, KVH, 256] with token stride ld_kv (elements,
 * multiple of 8), cos/sin fp16 [B, S, 256] ->
 *   k_rope fp16 [B, KVH, S, 256] (RoPE applied: the key states a KV cache stores) and
 *   kv_mfma, pi05w4a4_attn_kv_mfma_elems(B, S, KVH, 256) fp16 elements: per (b, KV head),
 *   K with RoPE and then V^T in MFMA-fragment-major order with the keys zero-padded to
 *   s_pad = S rounded up to 64 (K fragment (j, t), 512 elements at (8j + t) * 512: lane L
 *   holds K[16j + L%16][32t + 8(L/16) + 0..7]; V^T fragment (db, t) at
 *   s_pad*256 + (db*s_pad/32 + t) * 512: lane L holds V[32t + 8(L/16) + 0..7][16db + L%16]).
 * pi05w4a4_prefix_attention: q fp16 [B, S, H, 256] (token stride ld_q, the QKV GEMM's q
 * output; RoPE is applied inside), kv_mfma from kv_prep, the same cos/sin, an
 * optional additive fp16 mask (element (b, sq, sk) at mask[b*mask_bs + sq*mask_rs + sk];
 * mask_bs = 0 broadcasts one mask; mask_len >= S keys per row, a multiple of 4, strides
 * multiples of 4, 8-byte aligned; null for none) and `scaling` ->
 *   out fp16 [B, S, H, 256] with token stride ld_out (multiple of 4), or null, and
 *   with KVH == 1 and H == 8 optionally q_codes / q_scales: the o-proj input's K = 2048
 *   activation quant of the output rows (M = B * S, pi05w4a4_q_words(M, 2048) words and M
 *   scales, exactly what pi05w4a4_quantize writes for them), which replaces the
 *   quantize_x of the following int4_gemm (int4_gemm.cu:496-531); null for none.
 * All other pointers 16-byte aligned (out 8-byte).
 */
size_t pi05w4a4_attn_kv_mfma_elems(int64_t b, int32_t s, int32_t kvh, int32_t d);
int pi05w4a4_attn_kv_prep(const void* k, const void* v, int64_t ld_kv, const void* cos_fp16,
                          const void* sin_fp16, int64_t b, int32_t s, int32_t kvh, int32_t d,
                          void* k_rope, void* kv_mfma, void* stream);
int pi05w4a4_prefix_attention(const void* q, int64_t ld_q, const void* kv_mfma,
                              const void* cos_fp16, const void* sin_fp16, const void* mask,
                              int64_t mask_bs, int64_t mask_rs, int32_t mask_len, float scaling,
                              int64_t b, int32_t s, int32_t h, int32_t kvh, int32_t d, void* out,
                              int64_t ld_out, int32_t* q_codes, float* q_scales, void* stream);

/*
 * QKV GEMMs with the attention prep in the epilogue (one KV head of 256): pi05w4a4_gemm_multi
 * of the three weights, where the K output goes through RoPE and both K and V are also
 * written in the fragment-major layout pi05w4a4_attn_kv_prep produces, so that
 * pi05w4a4_prefix_attention follows with no kv_prep launch.  No counterpart in the
 * reference (its attention runs transformers' RoPE and eager attention after the
 * int4_gemm3 of apply.py:145-191); the fused decoder layer of this package uses it.
 *   w_k_rope: the K weight (MFMA layout, N = 256) with its 16-row blocks in RoPE-pair order
 *     (block 2P + j holds output channels 16P + 128j .. + 15, P < 8; pi05w4a4_permute_rope_pairs);
 *   cos_fp16 / sin_fp16: fp16 [B * S, 256] rotary tables of the rows;
 *   y_q fp16 [M, n_q]; k_rope fp16 [M, 256] (the key states with RoPE, dimension order);
 *   y_v fp16 [M, 256]; kv_mfma: pi05w4a4_attn_kv_mfma_elems(B, S, 1, 256) elements, pad keys
 *   zeroed.  M = B * S with S a multiple of 8 and at most 1024.  The whole K runs in one
 *   launch (no global K split, so no workspace), also where pi05w4a4_gemm_multi would split.
 */
int pi05w4a4_gemm_qkv_rope(const int32_t* q, const float* sa, int64_t m, int32_t k,
                           const int32_t* w_q_mfma, int32_t n_q, const int32_t* w_k_rope,
                           const int32_t* w_v_mfma, const void* cos_fp16, const void* sin_fp16,
                           int64_t b, int32_t s, void* y_q, void* k_rope, void* y_v, void* kv_mfma,
                           void* stream);

/*
 * The K weight of pi05w4a4_gemm_qkv_rope from an MFMA-layout K weight (N = 256, any K):
 * 16-row block 2P + j of dst is block P + 8j of src, with its scales and corrections.
 * dst holds pi05w4a4_mfma_words(256, K) words (a [256, K/8 + 16] tensor); not in place.
 */
int pi05w4a4_permute_rope_pairs(const int32_t* src_mfma, int32_t k, int32_t* dst_mfma, void* stream);

/*
 * pi05w4a4_prefix_attention plus cache warming: the CUs that the attention leaves idle
 * (B * KVH * ceil(S * H / KVH / 32) < 256 workgroups) read warm_n <= 4 further device
 * buffers (16-byte aligned, sizes multiples of 16 bytes) and discard the data, so that the
 * kernels after it find them in the Infinity Cache.  No counterpart in the reference: the
 * fused decoder layer passes its o-proj and MLP weights (o, gate, up, down), which the o,
 * gate/up and down GEMMs then read from the cache instead of HBM.  Results are those of
 * pi05w4a4_prefix_attention.
 */
int pi05w4a4_prefix_attention_warm(const void* q, int64_t ld_q, const void* kv_mfma,
                                   const void* cos_fp16, const void* sin_fp16, const void* mask,
                                   int64_t mask_bs, int64_t mask_rs, int32_t mask_len, float scaling,
                                   int64_t b, int32_t s, int32_t h, int32_t kvh, int32_t d, void* out,
                                   int64_t ld_out, int32_t* q_codes, float* q_scales,
                                   const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                                   void* stream);

/*
 * E3M2 operand form of the gate/up GEMM.  The same INT4 codes, held on the device as OCP
 * FP6 E3M2 values (every integer in [-8, 8] is one), feed gfx950's
 * v_mfma_f32_16x16x128_f8f6f4: half the int8 MFMA's issue time for the same work and no
 * nibble unpack; its fp32 sums of integer products stay below 2^24, so they equal the int32
 * accumulators of pi05w4a4_gemm bit for bit and every output is the same fp16 value.  An
 * alternative on-device form of the reference's int4_gemm2 / int4_gemm2_tiled for its
 * gate/up weights (int4_gemm.cu:533-564, 618-642; apply.py:135-138); no other counterpart.
 *   q6   activation codes, one 1536-byte fragment per 16 rows x 128 k: fragment (mb, kb) at
 *        byte (mb*KB + kb)*1536 (KB = K/128); bytes [0, 1024) hold dwords 0-3 of lane L at
 *        16 L, bytes [1024, 1536) dwords 4-5 of lane L at 1024 + 8 L, where lane L's six
 *        dwords hold codes 128 kb + 32 (L/16) .. +31 of row 16 mb + L%16, code j in bits
 *        6j .. 6j+5 (E3M2: sign bit 5, exponent bits 4-2 with bias 3, mantissa bits 1-0).
 *        pi05w4a4_q_e3m2_bytes(M, K) bytes, 16-byte aligned; no row corrections.
 *   w6   weights, int32 [N, 3K/16 + 16] (pi05w4a4_e3m2_words(N, K) words used): column
 *        pair p (columns 32p .. 32p+31) and k block kb form 3072 bytes at (p*KB + kb)*3072,
 *        three 1 KB chunks; chunk c holds bytes 16c .. 16c+15 of lane L's 48-byte record
 *        [six dwords of column 32p + L%16 | six dwords of column 32p + 16 + L%16] (codes
 *        as in q6) at 16 L.  The N fp32 column scales follow at word N*KB*24.
 * Shapes: K = 2048 for the quantizers (the gate/up input); K % 128 == 0, K <= 2^18 for the
 * GEMM; N % 32 == 0.
 *
 * pi05w4a4_repack_weight_e3m2: an MFMA-layout weight (pi05w4a4_repack_weight's output) ->
 *   w6, not in place (load time).
 * pi05w4a4_quantize_e3m2 / pi05w4a4_rmsnorm_quantize_e3m2: pi05w4a4_quantize /
 *   pi05w4a4_rmsnorm_quantize with the codes written as q6 (the same codes and scales).
 * pi05w4a4_rmsnorm_quantize_e3m2_warm: pi05w4a4_rmsnorm_quantize_e3m2 with the cache
 *   warming of pi05w4a4_rmsnorm_quantize_warm (the gate/up op passes part of its up weight).
 * pi05w4a4_gemm_e3m2: gelu_up = 0: pi05w4a4_gemm_multi of 1..3 w6 weights (n[g] columns
 *   into y[g]); gelu_up = 1: pi05w4a4_gemm_gelu_up (ngroups = 2: gate, up with
 *   n[0] == n[1]; y[0] = fp16(gelu_tanh(gate) * up)).  One launch, no workspace.
 */
size_t pi05w4a4_q_e3m2_bytes(int64_t m, int32_t k);
size_t pi05w4a4_e3m2_words(int32_t n, int32_t k);
int pi05w4a4_repack_weight_e3m2(const int32_t* w_mfma, int32_t n, int32_t k, int32_t* w6, void* stream);
int pi05w4a4_quantize_e3m2(const void* x_fp16, int64_t m, int32_t k, void* q6, float* sa, void* stream);
int pi05w4a4_rmsnorm_quantize_e3m2(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                   int64_t m, int32_t k, void* q6, float* sa, void* stream);
int pi05w4a4_rmsnorm_quantize_e3m2_warm(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                        int64_t m, int32_t k, void* q6, float* sa, const void* const* warm_ptrs,
                                        const size_t* warm_bytes, int32_t warm_n, void* stream);
int pi05w4a4_gemm_e3m2(const void* q6, const float* sa, int64_t m, int32_t k, int32_t ngroups,
                       const int32_t* const* w6, const int32_t* n, void* const* y_fp16, int32_t gelu_up,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PI05_W4A4_H_ */
