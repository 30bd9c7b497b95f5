/*
 * mk_hip.h -- C ABI of libmk_hip.so, the MI355X (gfx950) implementation of the
 * quantized decode hot path of manishklach/mlx-metal-kernels.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and a hipStream_t (passed as
 *     void*; NULL = the legacy default stream), launches asynchronously on that
 *     stream and never synchronizes;
 *   - returns MK_OK (0) or a negative status: MK_ERR_INVALID for a rejected
 *     argument (checked before anything is launched), MK_ERR_UNSUPPORTED for a
 *     shape/dtype combination no kernel handles, or -(1000 + hipError_t) when
 *     the launch itself failed;
 *   - allocates nothing: outputs and workspaces are owned by the caller.
 *
 * Layouts are row-major and dense (C-contiguous).  Activations are fp16 or
 * bf16 (MK_DT_F16 / MK_DT_BF16); quantization scales/zeros are fp16 or fp32.
 * Positions, lengths and block tables are int32.
 *
 * Each declaration names the reference function it replaces
 * (/root/reference paths, file:line).
 */
#ifndef MK_HIP_H_
#define MK_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MK_OK 0
#define MK_ERR_INVALID (-1)
#define MK_ERR_UNSUPPORTED (-2)
/* mk_paged_decode_attention_noalloc only: the call needs more scratch than
 * the library's fixed no-allocation buffer holds. */
#define MK_ERR_SCRATCH (-3)

#define MK_DT_F16 0
#define MK_DT_BF16 1
#define MK_DT_F32 2

/* IEEE binary16 value held as its raw bits (quantized-KV scales). */
typedef uint16_t f16_storage_t;

/* ABI version; bumped when entry points are added or their signatures change. */
int mk_abi_version(void);

/* ---------------------------------------------------------------- q4/q8 pack / dequant */

/* pack_q4 -- ops/quant_ops.py:166-176.  q [rows,K] codes 0..15 ->
 * packed [rows, ceil(K/2)], low nibble = even column, odd K padded with 0. */
int mk_pack_q4(const uint8_t* q, uint8_t* packed, int64_t rows, int64_t K, void* stream);

/* unpack_q4_reference -- ops/quant_ops.py:179-188.  packed [rows,Kp] ->
 * q [rows,K_out] with K_out <= 2*Kp. */
int mk_unpack_q4(const uint8_t* packed, uint8_t* q, int64_t rows, int64_t k_packed, int64_t k_out,
                 void* stream);

/* dequant_q4 -- ops/quant_ops.py:215-253 (kernels/dequant_q4.metal).
 * out[r,k] = (q - zeros[r,k/g]) * scales[r,k/g] in fp32, rounded to out_dtype;
 * zeros == NULL means z = 0.  K = 2*k_packed. */
int mk_dequant_q4(const uint8_t* packed, const void* scales, const void* zeros, void* out,
                  int64_t rows, int64_t k_packed, int64_t group_size, int scale_dtype,
                  int out_dtype, void* stream);

/* dequant_q8 -- ops/quant_ops.py:279-316 (kernels/dequant_q8.metal). */
int mk_dequant_q8(const uint8_t* q, const void* scales, const void* zeros, void* out, int64_t rows,
                  int64_t K, int64_t group_size, int scale_dtype, int out_dtype, void* stream);

/* quantize_weight_groupwise -- models/quantize_weights.py:164-203 (symmetric):
 * weight [rows, K] (fp32/fp16/bf16) -> codes uint8 [rows, ceil(K/2)] (q4,
 * low nibble = even k, odd K padded with 0) or [rows, K] (q8), and scales
 * [rows, ceil(K/g)] in scale_dtype.  scale = max(max|w| / (7|127), eps) in
 * double, codes = clip(rint(w / float(scale)), -limit, limit) + 8|128. */
int mk_quantize_weight(const void* weight, uint8_t* codes, void* scales, int64_t rows, int64_t K,
                       int64_t group_size, int bits, double eps, int w_dtype, int scale_dtype,
                       void* stream);

/* ---------------------------------------------------------------- quantized matvec family */

/* q4_matvec_decode -- ops/quant_ops.py:529-571 (all four backends:
 * metal / metal_parallel / metal_tiled / auto).
 * x [M,K] act_dtype, w [N, ceil(K/2)] packed q4, scales/zeros [N, ceil(K/g)]
 * scale_dtype (zeros nullable), y [M,N] act_dtype = saturate(x @ dequant(w)^T).
 * residual (nullable, [M,N] act_dtype) adds an epilogue: when given, y_out
 * receives residual + round(x @ W^T) (ops/mlp_block_ops.py:361) and y_mm
 * (nullable) the plain product. */
int mk_q4_matvec(const void* x, const uint8_t* w, const void* scales, const void* zeros,
                 const void* residual, void* y_mm, void* y_out, int64_t M, int64_t N, int64_t K,
                 int64_t group_size, int act_dtype, int scale_dtype, void* stream);

/* q8_matvec_decode -- ops/quant_ops.py:591-631.  w [N,K] uint8. */
int mk_q8_matvec(const void* x, const uint8_t* w, const void* scales, const void* zeros,
                 const void* residual, void* y_mm, void* y_out, int64_t M, int64_t N, int64_t K,
                 int64_t group_size, int act_dtype, int scale_dtype, void* stream);

/* q4_gate_up_matvec_tiled -- ops/quant_ops.py:634-685 (one x read, two weight
 * streams).  gate_out/up_out [M,N] (nullable) receive the two products;
 * mlp_out [M,N] (nullable) receives the fused SwiGLU epilogue
 * silu(gate)*up (ops/activation_ops.py:83-88) computed from the rounded
 * gate/up values.  At least one output must be non-NULL. */
int mk_q4_gate_up(const void* x, const uint8_t* w_gate, const uint8_t* w_up,
                  const void* s_gate, const void* s_up, const void* z_gate, const void* z_up,
                  void* gate_out, void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K,
                  int64_t group_size, int act_dtype, int scale_dtype, void* stream);

/* q8_gate_up_matvec_tiled -- ops/quant_ops.py:688-738. */
int mk_q8_gate_up(const void* x, const uint8_t* w_gate, const uint8_t* w_up,
                  const void* s_gate, const void* s_up, const void* z_gate, const void* z_up,
                  void* gate_out, void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K,
                  int64_t group_size, int act_dtype, int scale_dtype, void* stream);

/* The front of quantized_mlp_block -- ops/mlp_block_ops.py:343-356: residual
 * add z = x + residual (z_out [M,K]), RMSNorm normed = z * rsqrt(mean(z^2) +
 * eps) * norm_w (normed_out [M,K]), then the gate/up products and SwiGLU as
 * mk_q4_gate_up / mk_q8_gate_up.  For q4 or q8 with an M = 1 fp16 row, K <=
 * 8192, fp16 norm weights and fp16 scales this is one launch (the norm runs inside
 * the gate/up kernel) and normed_out may be NULL; otherwise the norm kernel
 * and the gate/up kernel run in turn through normed_out, which is then
 * required (MK_ERR_INVALID when NULL).
 * norm_w_dtype: MK_DT_F16/BF16/F32. */
int mk_q4_rmsnorm_gate_up(const void* x, const void* residual, const void* norm_w, float eps,
                          const uint8_t* w_gate, const uint8_t* w_up, const void* s_gate, const void* s_up,
                          const void* z_gate, const void* z_up, void* z_out, void* normed_out, void* gate_out,
                          void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K, int64_t group_size,
                          int act_dtype, int scale_dtype, int norm_w_dtype, void* stream);

int mk_q8_rmsnorm_gate_up(const void* x, const void* residual, const void* norm_w, float eps,
                          const uint8_t* w_gate, const uint8_t* w_up, const void* s_gate, const void* s_up,
                          const void* z_gate, const void* z_up, void* z_out, void* normed_out, void* gate_out,
                          void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K, int64_t group_size,
                          int act_dtype, int scale_dtype, int norm_w_dtype, void* stream);

/* RMSNorm + q4/q8 matvec: y = (x * rsqrt(mean(x^2) + eps) * norm_w, rounded
 * to the activation dtype) . W^T -- the input norm and qkv projection of the
 * decode layer (ops/llama_layer_ops.py:256-260 + ops/quantized_decode_block_ops.py:
 * 154-184) and the final norm and head of the stack (ops/llama_stack_ops.py:
 * 396-405).  x [M,K]; weights as mk_q4_matvec / mk_q8_matvec; y [M,N].
 * For q4 with an M = 1 fp16 row, K <= 8192, fp16 norm weights and fp16
 * scales this is one launch and normed_out [M,K] may be NULL; otherwise the
 * norm kernel writes normed_out (then required) and the matvec reads it. */
int mk_q4_rmsnorm_matvec(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                         const void* zeros, void* normed_out, void* y, int64_t M, int64_t N, int64_t K,
                         int64_t group_size, int act_dtype, int scale_dtype, int norm_w_dtype, void* stream);

int mk_q8_rmsnorm_matvec(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                         const void* zeros, void* normed_out, void* y, int64_t M, int64_t N, int64_t K,
                         int64_t group_size, int act_dtype, int scale_dtype, int norm_w_dtype, void* stream);

/* A decode layer's front half up to attention, in one launch where it can:
 * RMSNorm (ops/llama_layer_ops.py:256-258) + qkv projection
 * (ops/quantized_decode_block_ops.py:154-184) + GQA split + interleaved RoPE
 * + paged K/V write of the new token (ops/gqa_ops.py:493-547, as
 * mk_qkv_rope_paged_update).  x [M, K]; w [(Hq + 2 Hkv) D, K] packed; the
 * rounding of every stage is that of mk_q*_rmsnorm_matvec followed by
 * mk_qkv_rope_paged_update, so q_out and the caches match that pair exactly.
 * One launch for q4 fp16 (activations, scales, norm weight, pages) with
 * M == 1 and K <= 8192; for other fp16 batches the norm kernel writes
 * normed_out [M, K] and the projection's epilogue rotates and writes (two
 * launches); otherwise the projection goes through qkv_scratch [M, (Hq +
 * 2 Hkv) D] and then mk_qkv_rope_paged_update.  qkv_scratch must be given
 * (written only on that last path); normed_out is required unless the
 * one-launch path applies.  K/V pages carry the activation dtype. */
int mk_q4_rmsnorm_qkv_rope_paged(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                                 const void* zeros, void* qkv_scratch, void* normed_out, const float* cos_t,
                                 const float* sin_t, const int32_t* positions, const int32_t* block_table,
                                 void* K_pages, void* V_pages, void* q_out, int64_t M, int64_t Hq, int64_t Hkv,
                                 int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                 int64_t cos_rows, int64_t K, int64_t group_size, int act_dtype, int scale_dtype,
                                 int norm_w_dtype, void* stream);

int mk_q8_rmsnorm_qkv_rope_paged(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                                 const void* zeros, void* qkv_scratch, void* normed_out, const float* cos_t,
                                 const float* sin_t, const int32_t* positions, const int32_t* block_table,
                                 void* K_pages, void* V_pages, void* q_out, int64_t M, int64_t Hq, int64_t Hkv,
                                 int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                 int64_t cos_rows, int64_t K, int64_t group_size, int act_dtype, int scale_dtype,
                                 int norm_w_dtype, void* stream);

/* ---------------------------------------------------------------- elementwise / norm */

/* greedy_sample -- models/sampling.py:120-124 (np.argmax per row): out[r] = the
 * index of the largest of x[r, 0..n), the first on ties, a NaN counting as
 * the largest.  x [rows, n] f16/bf16/f32 (dtype), out int64 [rows]. */
int mk_argmax_rows(const void* x, int64_t* out, int64_t rows, int64_t n, int dtype, void* stream);


/* swiglu / fused_swiglu -- ops/activation_ops.py:91-153.
 * out = gate / (1 + exp(-gate)) * up, fp32 math, n elements. */
int mk_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/* residual_add -- ops/fused_ops.py:155-180.  out = x + residual in fp32. */
int mk_residual_add(const void* x, const void* residual, void* out, int64_t n, int dtype,
                    void* stream);

/* rms_norm -- ops/norm_ops.py:55-85.  y = x * rsqrt(mean(x^2) + eps) * w
 * over rows of length D; w_dtype may differ from x_dtype (fp16/bf16/fp32). */
int mk_rms_norm(const void* x, const void* weight, void* y, int64_t rows, int64_t D, float eps,
                int x_dtype, int w_dtype, void* stream);

/* residual_add + rms_norm as one pass (prologue of
 * ops/mlp_block_ops.py:343-344): z = x + residual, y = rms_norm(z, w). */
int mk_residual_rms_norm(const void* x, const void* residual, const void* weight, void* z_out,
                         void* y_out, int64_t rows, int64_t D, float eps, int x_dtype,
                         int w_dtype, void* stream);

/* ---------------------------------------------------------------- paged KV plumbing */

/* block_table_lookup -- ops/paged_kv_ops.py:155-182 (kernels/block_table_lookup.metal).
 * page_ids[b] = bt[b, pos[b]/P], offsets[b] = pos[b] % P. */
int mk_block_table_lookup(const int32_t* block_table, const int32_t* positions, int32_t* page_ids,
                          int32_t* offsets, int64_t B, int64_t max_blocks, int64_t page_size,
                          void* stream);

/* paged_kv_cache_update -- ops/paged_kv_ops.py:216-255, done in place:
 * K_pages/V_pages [num_pages,P,H,D] get k_new/v_new [B,H,D] written into slot
 * (bt[b,pos/P], pos%P).  A later b wins on a collision.  Out-of-range
 * positions or page ids are skipped. */
int mk_paged_kv_update(void* K_pages, void* V_pages, const void* k_new, const void* v_new,
                       const int32_t* block_table, const int32_t* positions, int64_t B, int64_t H,
                       int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                       int dtype, void* stream);

/* Fused GQA qkv split + interleaved RoPE + paged KV update for one decode
 * token -- composition of ops/gqa_ops.py:148-160 (reference_gqa_qkv_split_rope),
 * ops/rope_ops.py:61-75 and ops/paged_kv_ops.py:185-213, as
 * paged_gqa_decode_block_from_qkv (ops/gqa_ops.py:493-547) runs them.
 * qkv [B, (Hq+2*Hkv)*D]; cos/sin [cos_rows, D/2] fp32; q_out [B,Hq,D]. */
int mk_qkv_rope_paged_update(const void* qkv, const float* cos_t, const float* sin_t,
                             const int32_t* positions, const int32_t* block_table, void* K_pages,
                             void* V_pages, void* q_out, int64_t B, int64_t Hq, int64_t Hkv,
                             int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                             int64_t cos_rows, int dtype, void* stream);

/* Same, writing the new token into a symmetric q8/q4 paged cache
 * (ops/paged_quantized_kv_ops.py:146-175 quantizers; no reference kernel
 * exists for this write).  K_q/V_q [num_pages,P,Hkv,D] (q8) or [...,ceil(D/2)]
 * (q4) uint8; K_s/V_s [num_pages,P,Hkv,ceil(D/g)] fp16. */
int mk_qkv_rope_paged_update_quant(const void* qkv, const float* cos_t, const float* sin_t,
                                   const int32_t* positions, const int32_t* block_table,
                                   uint8_t* K_q, uint8_t* V_q, f16_storage_t* K_s,
                                   f16_storage_t* V_s, void* q_out, int64_t B, int64_t Hq,
                                   int64_t Hkv, int64_t D, int64_t page_size, int64_t max_blocks,
                                   int64_t num_pages, int64_t cos_rows, int64_t group_size,
                                   int bits, int dtype, void* stream);

/* quantize_kv_pages -- ops/paged_quantized_kv_ops.py:194-292 for one of K or V:
 * src [rows, D] (rows = num_pages*P*Hkv) -> codes [rows, D] (q8) or
 * [rows, ceil(D/2)] (q4) and fp16 scales [rows, ceil(D/g)], with the
 * quantizer of :146-175 (correctly rounded fp32 divide, round half to even). */
int mk_quantize_kv(const void* src, uint8_t* codes, f16_storage_t* scales, int64_t rows, int64_t D,
                   int64_t group_size, int bits, int dtype, void* stream);

/* ---------------------------------------------------------------- paged decode attention */

/* Workspace (bytes, 16-byte aligned) the split-context attention kernels
 * need for B sequences of at most max_blocks pages, Hq query / Hkv key-value
 * heads of dimension D, on the current device.  Its first 128 KiB hold
 * arrival counters: fill the workspace with zeros once, before its first
 * call; every call leaves the counters zero again, so the buffer can then be
 * reused without clearing (the rest holds split partials, any content).
 * Calls that may run concurrently need distinct workspaces.  No reference
 * counterpart: the reference's one-thread-per-head kernels do not split the
 * context. */
size_t mk_paged_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                          int64_t max_blocks, int64_t page_size);

/* Paged GQA/MQA/MHA decode attention over an fp16/bf16 paged cache --
 * reference_paged_gqa_decode_attention (ops/gqa_ops.py:307-342) and
 * paged_decode_attention (ops/paged_kv_ops.py:307-360, the Hq == Hkv case).
 * q [B,Hq,D]; K/V_pages [num_pages,P,Hkv,D]; bt [B,max_blocks]; lengths [B]
 * (clipped to max_blocks*P); out [B,Hq,D].  Length 0 yields zeros. */
int mk_paged_decode_attention(const void* q, const void* K_pages, const void* V_pages,
                              const int32_t* block_table, const int32_t* lengths, void* out,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                              int64_t max_blocks, int64_t num_pages, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream);

/* mk_paged_decode_attention without a workspace argument.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split partials and arrival counters live in a fixed
 * 16 MiB device array inside the library (zero when the library loads, one
 * per device, held until the process ends); a shape whose
 * partials exceed it returns MK_ERR_SCRATCH before anything is launched
 * (config 3 needs 4.5 MiB).  The call allocates nothing.  Calls on one device
 * share that array, so calls that overlap in time on one device (different
 * streams, or host threads) race; serialise them on one stream.  The current
 * device must be the device of q and of the stream. */
int mk_paged_decode_attention_noalloc(const void* q, const void* K_pages, const void* V_pages,
                                      const int32_t* block_table, const int32_t* lengths,
                                      void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                      float scale, int dtype, void* stream);

/* paged_quantized_kv_gqa_decode_attention -- ops/paged_quantized_kv_ops.py:632-661
 * (kernels/q8_paged_gqa_decode_attention.metal, q4_...).  Codes/scales as in
 * mk_qkv_rope_paged_update_quant; page ids < 0 are skipped. */
int mk_paged_quantized_decode_attention(const void* q, const uint8_t* K_q, const uint8_t* V_q,
                                        const f16_storage_t* K_s, const f16_storage_t* V_s,
                                        const int32_t* block_table, const int32_t* lengths,
                                        void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                        int64_t group_size, int bits, float scale, int dtype,
                                        void* workspace, size_t workspace_bytes, void* stream);

/* Speculative-verify attention: W draft rows per sequence in one pass over
 * the cache -- the attention of the staged verify loop
 * (ops/speculative_verify_ops.py:228-262, each step a paged GQA decode,
 * ops/gqa_ops.py:307-342).  q and out [B, W, Hq, D]; lengths [B] count the
 * context and all W new positions; row w sees positions
 * < lengths[b] - (W - 1 - w) (none: zeros).  The W * Hq/Hkv rows of one kv
 * head are the columns of one MFMA contraction, so each K/V byte is read
 * once for all W rows.  Workspace: mk_paged_attention_workspace_bytes(B,
 * W * Hq, Hkv, D, max_blocks, page_size).  1 <= W <= 64. */
int mk_paged_verify_attention(const void* q, const void* K_pages, const void* V_pages,
                              const int32_t* block_table, const int32_t* lengths, void* out,
                              int64_t B, int64_t W, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                              int64_t max_blocks, int64_t num_pages, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream);

/* mk_paged_verify_attention over q8/q4 pages (layout as
 * mk_paged_quantized_decode_attention). */
int mk_paged_quantized_verify_attention(const void* q, const uint8_t* K_q, const uint8_t* V_q,
                                        const f16_storage_t* K_s, const f16_storage_t* V_s,
                                        const int32_t* block_table, const int32_t* lengths, void* out,
                                        int64_t B, int64_t W, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                        int64_t group_size, int bits, float scale, int dtype,
                                        void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MK_HIP_H_ */
