/* C ABI of libdk.so: the gfx950 kernels of the NF4 QLoRA linear path.
 *
 * Conventions (the reference's operator conventions, solution/k_nf4.py:176-205,
 * solution/k_mlp.py:50-63):
 *   - every pointer is a device pointer into caller-allocated memory; nothing is allocated here;
 *   - every launch is asynchronous on `stream` (a hipStream_t; 0 = the null stream);
 *   - fp16 tensors are passed as void* (IEEE binary16), row-major and contiguous unless a leading
 *     dimension is given;
 *   - return 0 on success, a negative DK_ERR_* for an argument error detected before any launch,
 *     or a positive hipError_t from the launch;
 *   - no mutable global state (only once-filled per-device caches: the CU count, the address of
 *     the allocation-free entry point's device array): entry points may be called from any host
 *     thread; every choice a call makes comes from its own arguments.
 */
#ifndef DK_H
#define DK_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DK_ERR_INVALID (-1)   /* a size or a null pointer that the operation cannot accept */
#define DK_ERR_ALIGN (-2)     /* a pointer or an offset breaks the alignment the kernel needs */
#define DK_ERR_WORKSPACE (-3) /* the workspace is missing or too small */
#define DK_ERR_CAPTURE (-4)   /* a one-time set-up that cannot run under stream capture is still
                                 due: make the same call once outside capture first */

/* An NF4 double-quantised weight [rows, cols] (out_features x in_features), element
 * e = row * cols + col.  The four sections are those of the reference's repacked layer
 * (solution/k_nf4.py:64-95): packed nibbles (even element in the high nibble), one uint8 code
 * per 64 weights, one fp32 scale and one fp32 offset per 16384 weights.  code2 is the 256-entry
 * second-level code table and nf4 the 16-entry NF4 table, both fp32. */
typedef struct dk_nf4_weight {
  const uint8_t* packed;  /* [rows * cols / 2]     */
  const uint8_t* qabs;    /* [rows * cols / 64]    */
  const float* scale2;    /* [rows * cols / 16384] */
  const float* offset2;   /* [rows * cols / 16384] */
  const float* code2;     /* [256] */
  const float* nf4;       /* [16]  */
  int64_t rows;
  int64_t cols;
  int32_t kernel;         /* DK_W4_KERNEL_*: which GEMM kernel the dk_w4_* calls on this weight
                             run (0, the default, lets the library choose) */
} dk_nf4_weight;

/* Values of dk_nf4_weight.kernel (no counterpart in the reference: its GEMMs read a dequantised
 * workspace).  The 256 x 256-tile kernel can read the packed NF4 weight itself, each workgroup
 * dequantising its W tiles into LDS (bit-identical to the fp16-weight form); otherwise the weight
 * is first dequantised into the workspace and read as fp16, or the 128 x 128 warp-specialised
 * kernel dequantises in LDS.  AUTO: the tile kernel reads NF4 where that is fastest (its split-K
 * plans: few output tiles, long K); TILE: wherever its plan takes the shape; STAGED: never.  The
 * choice travels with each call's weight argument: the library keeps no setting of its own. */
#define DK_W4_KERNEL_AUTO 0
#define DK_W4_KERNEL_TILE 1
#define DK_W4_KERNEL_STAGED 2

/* Human-readable text for a return code (static storage). */
const char* dk_error_string(int code);

/* ------------------------------------------------------------------------------------------
 * NF4 dequant.  Replaces k_nf4.dequant_tensors / nf4_layer_dequant_kernel
 * (solution/k_nf4.py:40-57, 176-181): out[e] = fp16(NF4[nib(e)] * absmax[e / 64]) for every
 * element of n_qblocks * 64, bit-exact.  packed and out must be 16-byte aligned. */
int dk_nf4_dequant(const uint8_t* packed, const uint8_t* qabs, const float* scale2,
                   const float* offset2, const float* code2, const float* nf4, void* out_f16,
                   int64_t n_qblocks, hipStream_t stream);

/* NF4 quantisation with double quantisation (blocksize 64, second level 256) of an fp16 weight.
 * Replaces the bitsandbytes quantisation the reference's weights come from (Params4bit with
 * quant_type="nf4", compress_statistics=True, blocksize=64; solution/test_kernels.py:46-56,
 * format checks solution/k_nf4.py:98-114).  numel % 16384 == 0.  absmax_ws: fp32
 * [numel / 64] scratch; sum_ws: one uint64 of scratch.  offset2 receives the weight's mean
 * offset, broadcast per second-level block (solution/k_nf4.py:168). */
int dk_nf4_quantize(const void* w_f16, int64_t numel, const float* code2, const float* nf4,
                    uint8_t* packed, uint8_t* qabs, float* scale2, float* offset2,
                    float* absmax_ws, uint64_t* sum_ws, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Gated SiLU on the fused [gate | up] rows.  Replace k_mlp.gated_silu_forward /
 * gated_silu_backward (solution/k_mlp.py:20-63): gu is [n_rows, 2 * inter] fp16.
 * forward:  act = fp16(silu(g) * u), act [n_rows, inter].
 * backward: gu <- [dact * u * sig * (1 + g * (1 - sig)) | dact * silu(g)], in place. */
int dk_gated_silu_fwd(const void* gu, void* act, int64_t n_rows, int64_t inter,
                      hipStream_t stream);
int dk_gated_silu_bwd(void* gu, const void* dact, int64_t n_rows, int64_t inter,
                      hipStream_t stream);

/* Example SwiGLU of the stock path (solution/swiglu.py:15-37), flat fp16 tensors of n elements:
 * out = gate * sigmoid(gate) * up; dgate, dup from grad. */
int dk_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, hipStream_t stream);
int dk_swiglu_bwd(const void* grad, const void* gate, const void* up, void* dgate, void* dup,
                  int64_t n, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * The producer and the consumer around the LoRA'd q/v linear.
 *
 * Fused residual add + RMSNorm + the two LoRA dropout inputs, one token row of d (4 <= d <= 4096,
 * d % 4 == 0) per wave.  Replaces rms_fwd_kernel / rms_forward (solution/k_norm.py:29-58,
 * 114-131): h = x [+ fp32(delta)] (xout = h if given), rstd = rsqrt(mean(h^2) + eps),
 * y = w * (h * rstd), y16 = fp16(y) (if y), xq/xv = fp16(keep ? y * keep_scale : 0) (if xq and
 * xv, which need the uint8 keep-masks mq/mv).  x, xout, w fp32 (16-byte aligned); delta, y, xq,
 * xv fp16 [n_rows, d] (8-byte aligned); rstd fp32 [n_rows]; NULL leaves an output unwritten. */
int dk_rms_fwd(const float* x, const void* delta, float* xout, const float* w, void* y,
               float* rstd, void* xq, void* xv, const uint8_t* mq, const uint8_t* mv,
               int64_t n_rows, int64_t d, float eps, float keep_scale, hipStream_t stream);

/* RMSNorm backward with the LoRA-A input gradients.  Replaces rms_bwd_kernel / rms_backward
 * (solution/k_norm.py:61-88, 134-150): dy = fp32(dy) * gscale[0] (dy fp16, or fp32 when dy_f32:
 * the q|k|v dX GEMM's fp32 output that already holds the masked LoRA terms)
 * [+ (mq ? fp32(lq) * keep_scale : 0) + (mv ? fp32(lv) * keep_scale : 0)], h = x [+ delta],
 * xh = h * rstd, g = dy * w, dx = (g - xh * mean(g * xh)) * rstd [+ dres]; out fp32 (may alias
 * dres), out16 = fp16(dx) if given.  gscale is a device pointer to one fp32. */
int dk_rms_bwd(const void* dy, int dy_f32, const float* gscale, const float* x,
               const void* delta, const float* w, const float* rstd, const float* dres, float* out, const void* lq,
               const void* lv, void* out16, const uint8_t* mq, const uint8_t* mv, int64_t n_rows,
               int64_t d, float keep_scale, hipStream_t stream);

/* QKV epilogue, forward, in place on the fused [n_rows, (nq + 2 nkv) hd] fp16 QKV buffer.
 * Replaces qkv_epilogue_fwd_kernel / qkv_epilogue_forward (solution/k_rope.py:23-61, 107-111):
 * q += lora_scale * lq, v += lora_scale * lv (fp32), then q and k heads rotated by
 * [x1 c - x2 s | x2 c + x1 s] with c, s = cos/sin_table[pos[row] * hd + j], j < hd / 2; every
 * product and sum rounded to fp32 on its own, the result once to fp16.  lq [n_rows, nq hd], lv
 * [n_rows, nkv hd] fp16; pos int32 [n_rows]; tables fp32 [positions, hd] (16-byte aligned);
 * hd % 8 == 0. */
int dk_qkv_epilogue_fwd(void* qkv, const void* lq, const void* lv, const int32_t* pos,
                        const float* cos_table, const float* sin_table, int64_t n_rows,
                        float lora_scale, int nq, int nkv, int hd, hipStream_t stream);

/* QKV epilogue, backward.  Replaces qkv_epilogue_bwd_kernel / qkv_epilogue_backward
 * (solution/k_rope.py:64-104, 114-119): out [n_rows, (nq + 2 nkv) hd] fp16 = [rot^T(dq) |
 * rot^T(sum of the gin partials of each KV head of dk) | sum of the gin partials of dv], with
 * rot^T: [d1 c + d2 s | d2 c - d1 s].  dq [n_rows, nq hd], dk/dv [n_rows, nkv gin hd], fp32
 * (grads_f32 != 0, 16-byte aligned) or fp16. */
int dk_qkv_epilogue_bwd(const void* dq, const void* dk, const void* dv, int grads_f32,
                        const int32_t* pos, const float* cos_table, const float* sin_table,
                        void* out, int64_t n_rows, int nq, int nkv, int hd, int gin,
                        hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Variable-length causal GQA attention of the packed batch (the consumer of the QKV epilogue).
 * qkv [n_tokens, (nq + 2 nkv) hd] fp16 as the QKV epilogue writes it; cu_seqlens [n_seq + 1]
 * int32; block_table: n_blocks (sequence, first row) int32 pairs, blocks of 128 rows that never
 * straddle two sequences (k_attn.block_table(lens, 128)); hd = 128, nq % nkv == 0.  Scores use
 * the scale log2(e) / sqrt(hd) in the exp2 domain.
 * dk_attn_fwd replaces attention_forward (solution/k_attn.py:40-83, 202-212): out
 * [n_tokens, nq hd] fp16, lse [nq, n_tokens] fp32 = m + log2(l) per (head, token).
 * dk_attn_bwd replaces attention_backward (solution/k_attn.py:84-182, 215-245): delta
 * [nq, n_tokens] fp32 scratch, dq [n_tokens, nq hd] fp32, dkp / dvp [n_tokens, nq hd] fp32
 * per-query-head partials (dk_qkv_epilogue_bwd with gin = nq / nkv sums them).  Any order of
 * the block table gives the same results; ordered by the rows from a block's start to its
 * sequence's end, longest first (k_attn.bwd_block_table), the launch balances best.  Requires
 * 2 n_blocks nq < 2^31 (DK_ERR_INVALID otherwise). */
int dk_attn_fwd(const void* qkv, const int32_t* cu_seqlens, int32_t n_seq,
                const int32_t* block_table, int32_t n_blocks, int64_t n_tokens, int32_t nq,
                int32_t nkv, int32_t hd, void* out, float* lse, hipStream_t stream);
int dk_attn_bwd(const void* qkv, const void* out, const float* lse, const void* dout,
                const int32_t* cu_seqlens, int32_t n_seq, const int32_t* block_table,
                int32_t n_blocks, int64_t n_tokens, int32_t nq, int32_t nkv, int32_t hd,
                float* delta, float* dq, float* dkp, float* dvp, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * LM head over vocabulary chunks (the consumer of the final norm): the row kernels between the
 * two GEMMs of each chunk (logits_c = Y E_c^T by dk_h16_linear_fwd_lora, acc += P E_c by
 * dk_h16_linear_bwd_dx_lora with DK_OUT_F32_ACCUM).  Rows are in sorted order (rows with a target
 * first, n_lab of them); state [n_rows, 8] fp32 = (m, s, t, argmax, x_target, pad), m = -inf and
 * the rest 0 before the first chunk; acc [n_lab, d] fp32 starts at 0.
 * dk_head_chunk replaces head_chunk_kernel (solution/k_head.py:50-123): logits [n_rows, vc] fp16
 * of chunk [v0, v0 + vc) (vc % 8 == 0, v0 + vc <= 2^24 so that the fp32 argmax is exact,
 * n_rows <= INT32_MAX), merged into the state; rows r < n_lab get
 * P = p_scale e^(x - m) in place (0 in the target's column) and their acc rows rescaled.
 * dk_head_finalize replaces head_finalize_kernel (solution/k_head.py:126-161): stats [n_rows, 4]
 * = (loss, entropy, hit, lse), and dy [n_rows, d] fp16 row perm[r] = out_scale (acc / (p_scale s)
 * + (p_target - 1) e_target[r]) for r < n_lab, 0 otherwise (inv_p_scale = 1 / p_scale). */
int dk_head_chunk(void* logits, const int32_t* tgt_sorted, float* state, float* acc,
                  int64_t n_rows, int64_t n_lab, int64_t vc, int64_t v0, float p_scale, int64_t d,
                  hipStream_t stream);
int dk_head_finalize(const float* state, const int32_t* tgt_sorted, const int32_t* perm,
                     const float* acc, const void* e_target, float* stats, void* dy,
                     int64_t n_rows, int64_t n_lab, float out_scale, float inv_p_scale, int64_t d,
                     hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * LoRA down projection with the dropout of its input.  Replaces the norm kernel's dropout lines
 * and the lora_A GEMM (solution/k_norm.py:49-53; solution/fast_qwen.py:943-944):
 *   Xd = fp16(mask ? fp32(x) * keep_scale : 0),   z = fp16(Xd A^T)
 * x [m, k] fp16, mask [m, k] uint8 (nonzero = keep; NULL = no dropout), a [rank, k] fp16,
 * z [m, rank] fp16.  rank % 16 == 0, rank <= 64, k % 32 == 0. */
int dk_lora_down(const void* x, const uint8_t* mask, float keep_scale, const void* a, void* z,
                 int64_t m, int64_t k, int64_t rank, hipStream_t stream);

/* Fused NF4 linear forward: y = X W^T (+ bias) (+ lora_scale * (z B^T)), dequant in LDS.
 * Replaces torch.addmm on the dequantised workspace plus the LoRA-B GEMM and the epilogue's
 * LoRA add (solution/fast_qwen.py:945-947; solution/k_rope.py:39-43, 54-58), rounding like them:
 *   y = fp16(fp32(fp16(X W^T + bias)) + s * fp32(fp16(z B^T))).
 * x [m, w.cols] fp16 (row stride ldx elements), y [m, w.rows] fp16 (row stride ldy),
 * bias [w.rows] fp16 or NULL, z [m, rank] fp16 and lora_b [w.rows, rank] fp16, or both NULL.
 * w.rows % 64 == 0, w.cols % 64 == 0.
 * workspace: scratch of dk_w4_workspace(m, w, DK_OP_LINEAR_FWD) bytes, 256-byte aligned, for
 * the split-K partial tiles (a second launch on the same stream sums them in a fixed order and
 * runs the epilogue) and the two-phase fp16 weight; NULL runs in one phase without split-K.
 * Launches that overlap in time must not share it. */
int dk_w4_linear_fwd(const void* x, int64_t ldx, int64_t m, const dk_nf4_weight* w,
                     const void* bias, const void* z, const void* lora_b, int64_t rank,
                     float lora_scale, void* y, int64_t ldy, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/* One rank-r LoRA term of a fused linear (used by the *_lora entry points, at most two each).
 * Forward:  adds s * fp32(fp16(left right^T)) to output columns [col_begin, col_end) (multiples of
 *           32, disjoint between terms); left = z [m, rank], right = B [col_end - col_begin, rank],
 *           mask NULL, scale = s.
 * Backward: adds (mask ? fp32(fp16(left right)) * scale : 0) to every column of dX, terms in
 *           order; left = dz [m, rank], right = A [rank, w.cols], mask [m, w.cols] uint8 or NULL
 *           (no dropout: the term is added unscaled), scale = keep_scale; col_* ignored. */
typedef struct dk_lora_term {
  const void* left;
  const void* right;
  const uint8_t* mask;
  int64_t col_begin;
  int64_t col_end;
  float scale;
} dk_lora_term;

/* The fused linear forward with up to two LoRA terms on disjoint output-column ranges.  Replaces
 * the fused QKV projection: qkv = addmm(bias_qkv, x, W_qkv^T) with the q and v LoRA adds of
 * qkv_epilogue_forward (solution/fast_qwen.py:943-949; solution/k_rope.py:39-43, 54-58), w being
 * the q|k|v rows of the repacked layer.  Rounding per term as in dk_w4_linear_fwd, terms added in
 * order.  Other arguments and rules as dk_w4_linear_fwd. */
int dk_w4_linear_fwd_lora(const void* x, int64_t ldx, int64_t m, const dk_nf4_weight* w,
                          const void* bias, const dk_lora_term* terms, int n_terms,
                          int64_t rank, void* y, int64_t ldy, void* workspace,
                          int64_t workspace_bytes, hipStream_t stream);

/* Workspace of the fused NF4 GEMMs.  No counterpart in the reference (cuBLAS manages its own);
 * it stands in for the reference's fp16 dequant workspace (solution/fast_qwen.py:398-418).
 * It holds split-K partial tiles and, from 512 rows on for outputs of at least 1536 columns, the
 * weight dequantised to fp16 once per call (the "two-phase" path: dequant at HBM rate, then the
 * MFMA GEMM on fp16 W), which at many row tiles is faster than dequantising each W tile again for
 * every row tile.  Without a
 * workspace (NULL) every entry point still runs, in one phase with the dequant in LDS.
 * Bytes needed at m rows for operation op (0: none). */
#define DK_OP_LINEAR_FWD 0         /* dk_w4_linear_fwd, dk_w4_linear_fwd_lora */
#define DK_OP_LINEAR_BWD_DX 1      /* dk_w4_linear_bwd_dx, dk_w4_linear_bwd_dx_lora */
#define DK_OP_GATEUP_SWIGLU_FWD 2  /* dk_w4_gateup_swiglu_fwd */
#define DK_OP_DOWN_SWIGLU_BWD 3    /* dk_w4_down_swiglu_bwd */
int64_t dk_w4_workspace(int64_t m, const dk_nf4_weight* w, int op);

/* dk_w4_workspace(m, w, backward ? DK_OP_LINEAR_BWD_DX : DK_OP_LINEAR_FWD). */
int64_t dk_w4_linear_workspace(int64_t m, const dk_nf4_weight* w, int backward);

/* Output modes of the backward dX GEMM. */
#define DK_OUT_F16 0         /* dx is fp16, overwritten */
#define DK_OUT_F32 1         /* dx is fp32, overwritten */
#define DK_OUT_F32_ACCUM 2   /* dx is fp32, dx += result */

/* Fused NF4 linear backward to the input: dX = dY W with the transposed dequant done in LDS,
 * plus the LoRA input-gradient term through the dropout mask.  Replaces the dX GEMMs and the
 * LoRA dX lines (solution/fast_qwen.py:1310, 1320-1327, 1350, 1364, 1376-1377;
 * solution/k_norm.py:65-71):
 *   dX = fp32(fp16(dY W)) + (mask ? fp32(fp16(dz A)) * keep_scale : 0)
 * dy [m, w.rows] fp16 (row stride lddy), dx [m, w.cols] (row stride lddx) in out_mode,
 * dz [m, rank] fp16, lora_a [rank, w.cols] fp16 and mask [m, w.cols] uint8, or all NULL.
 * workspace as for dk_w4_linear_fwd, sized by dk_w4_workspace(m, w, DK_OP_LINEAR_BWD_DX). */
int dk_w4_linear_bwd_dx(const void* dy, int64_t lddy, int64_t m, const dk_nf4_weight* w,
                        const void* dz, const void* lora_a, int64_t rank, const uint8_t* mask,
                        float keep_scale, void* dx, int64_t lddx, int out_mode,
                        void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* The backward dX GEMM with up to two LoRA dX terms (each with its own dropout mask).  Replaces
 * dy1 = mm(dqkv, W_qkv) and the lq/lv adds of rms_backward (solution/fast_qwen.py:1364,
 * 1376-1380; solution/k_norm.py:64-70):
 *   dX = fp32(fp16(dY W)) + (mq ? fp32(fp16(dz_q A_q)) * ks : 0) + (mv ? ... : 0)
 * Other arguments and rules as dk_w4_linear_bwd_dx. */
int dk_w4_linear_bwd_dx_lora(const void* dy, int64_t lddy, int64_t m, const dk_nf4_weight* w,
                             const dk_lora_term* terms, int n_terms, int64_t rank, void* dx,
                             int64_t lddx, int out_mode, void* workspace,
                             int64_t workspace_bytes, hipStream_t stream);

/* LoRA parameter gradients and the LoRA-down gradient.  Replaces
 * solution/fast_qwen.py:1369-1374:
 *   dB = fp32(fp16(dY^T z)) * s              [w_rows, rank] fp32
 *   dz = fp16(fp16(dY B) * s)                [m, rank] fp16
 *   dA = fp32(fp16(dz^T Xd)), Xd as in dk_lora_down   [rank, k] fp32
 * dy [m, n_out] fp16 with row stride lddy (a column slice of dQKV: gq = qkv[:, :NQ*HD]),
 * z [m, rank], x [m, k], mask [m, k] (NULL = no dropout), lora_b [n_out, rank].
 * Every column sum runs over all m rows in a fixed order (deterministic); with m == 0, dA and dB
 * are written as zeros and dy, z, x, dz may be NULL.  ws / ws_bytes are accepted and unused: the
 * workspace query returns 0. */
int64_t dk_lora_grads_workspace(int64_t m, int64_t n_out, int64_t k, int64_t rank);
int dk_lora_grads(const void* dy, int64_t lddy, const void* z, const void* x, const uint8_t* mask,
                  float keep_scale, const void* lora_b, float lora_scale, int64_t m,
                  int64_t n_out, int64_t k, int64_t rank, float* da, float* db, void* dz,
                  void* ws, int64_t ws_bytes, hipStream_t stream);

/* One or two LoRA adapters in shared launches: the q and v adapters of the fused QKV projection
 * (solution/fast_qwen.py:943-944 forward, 1364-1380 backward), each term computed exactly as by
 * dk_lora_down / dk_lora_grads (same kernels, same summation order).  A term's input is the
 * call's x, or its own x when set: the reference's xq and xv, the norm's fp32 output dropped out
 * per adapter and rounded once (solution/k_norm.py:49-53), are two inputs with no mask.  No
 * counterpart in the reference as one call: it batches the per-adapter calls above. */
typedef struct dk_lora_down_term {
  const uint8_t* mask;  /* [m, k] keep-mask or NULL */
  float keep_scale;
  const void* a;        /* lora_A [rank, k] fp16 */
  void* z;              /* [m, rank] fp16 out */
  const void* x;        /* [m, k] fp16 input of this term, or NULL for the call's x */
} dk_lora_down_term;
int dk_lora_down_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                       const dk_lora_down_term* terms, int n_terms, hipStream_t stream);

typedef struct dk_lora_grads_term {
  const void* dy;       /* [m, n_out] fp16, row stride lddy (a column slice of dQKV) */
  int64_t lddy;
  int64_t n_out;
  const void* z;        /* [m, rank] fp16 */
  const void* lora_b;   /* [n_out, rank] fp16 */
  float lora_scale;
  const uint8_t* mask;  /* [m, k] keep-mask or NULL */
  float keep_scale;
  float* da;            /* [rank, k] fp32 out */
  float* db;            /* [n_out, rank] fp32 out */
  void* dz;             /* [m, rank] fp16 out */
  const void* x;        /* [m, k] fp16 input of this term (dA's operand), or NULL for the call's x */
} dk_lora_grads_term;
/* x may be NULL when every term has its own.  ws / ws_bytes are accepted and unused (the
 * workspace query returns 0). */
int64_t dk_lora_grads_multi_workspace(int64_t m, int64_t k, int64_t rank, const int64_t* n_outs,
                                      int n_terms);
int dk_lora_grads_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                        const dk_lora_grads_term* terms, int n_terms, void* ws, int64_t ws_bytes,
                        hipStream_t stream);

/* The first half of dk_lora_grads_multi, for a caller whose q|k|v dX GEMM carries the second
 * (dk_h16_linear_bwd_dx_lora_sums): dz of every term only, the row pass
 * dz = fp16(fp16(dY B) * s) (solution/fast_qwen.py:1370, 1373).  Arguments as
 * dk_lora_grads_multi; da and db are not written here. */
int dk_lora_dz_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                     const dk_lora_grads_term* terms, int n_terms, hipStream_t stream);

/* The second half: the column sums dB = fp32(fp16(dY^T z)) * s and dA = fp32(fp16(dz^T Xd)) of
 * the terms (solution/fast_qwen.py:1369, 1371), for dk_h16_linear_bwd_dx_lora_sums to carry.  The
 * same x, m, k, rank and terms as the dk_lora_dz_multi call that computed their dz, which must
 * come first in stream order.  With it, dA and dB are bit-identical to dk_lora_grads_multi's. */
typedef struct dk_side_lora_sums {
  const void* x;
  int64_t m, k, rank;
  const dk_lora_grads_term* terms;
  int32_t n_terms;
} dk_side_lora_sums;

/* gate|up as one NF4 GEMM with the gated-SiLU epilogue.  Replaces the gate and up GEMMs and
 * gated_silu_forward (solution/fast_qwen.py:1080-1108; solution/k_mlp.py:20-29):
 *   g = fp16(X Wg^T), u = fp16(X Wu^T), act = fp16(silu(g) * u)
 * w_gu is [2 * inter, k]: the gate rows then the up rows (the repacked layer's gate|up order,
 * solution/k_nf4.py:7-9).  act [m, inter]; gu_out [m, 2 * inter] receives [g | u] when not NULL
 * (the saved gate|up of the backward).  inter % 32 == 0, k % 64 == 0.  workspace as for
 * dk_w4_linear_fwd, sized by dk_w4_workspace(m, w_gu, DK_OP_GATEUP_SWIGLU_FWD), or NULL. */
int dk_w4_gateup_swiglu_fwd(const void* x, int64_t ldx, int64_t m, const dk_nf4_weight* w_gu,
                            void* act, void* gu_out, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream);

/* Down-projection backward fused with the gated-SiLU backward.  Replaces dact = dh W_d and
 * gated_silu_backward (solution/fast_qwen.py:1310-1312; solution/k_mlp.py:32-47):
 *   dact = fp16(dh W_d);  gu <- [dact * u * sig * (1 + g * (1 - sig)) | dact * silu(g)]
 * dh [m, w_down.rows] fp16, w_down [d_model, inter], gu [m, 2 * inter] in/out.  workspace as
 * for dk_w4_linear_fwd, sized by dk_w4_workspace(m, w_down, DK_OP_DOWN_SWIGLU_BWD), or NULL. */
int dk_w4_down_swiglu_bwd(const void* dh, int64_t lddh, int64_t m, const dk_nf4_weight* w_down,
                          void* gu, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * The same GEMMs and epilogues on a weight already dequantised to fp16 (w16 [rows][cols], stored
 * like the NF4 weight: [out, in], in contiguous, 16-byte aligned).  These are the reference's
 * GEMMs on its dequantised workspace (torch.mm/addmm on views filled by k_nf4.dequant_range on a
 * side stream ahead of use, solution/fast_qwen.py:694-756, 943-947, 1093-1112, 1310-1364).
 * Arguments, rounding and rules as the dk_w4_* entry point of the same name; workspace (split-K
 * partials only) sized by dk_h16_workspace, or NULL.
 *
 * `side` (or NULL) is dequant work the launch carries: the reference's ahead-of-use dequant
 * (k_nf4.dequant_range on dq_stream, solution/fast_qwen.py:729-731) done inside the GEMM launch
 * by `wgs` extra workgroups, which run on the CUs the GEMM's tiles leave idle, instead of on a
 * second stream.  It dequantises second-level blocks [sb0, sb1) of one repacked layer: the four
 * section pointers are the layer's (as dk_nf4_dequant takes them), and weight e of the layer goes
 * to out[e] (fp16, 16-byte aligned), so out is the base of a whole-layer fp16 buffer.  The work is
 * complete when the GEMM is (stream order); out must not overlap anything the GEMM reads or
 * writes.  Bit-identical to dk_nf4_dequant over the same blocks.  wgs = 0 or sb0 = sb1: none.
 * GEMMs that the 256 x 256-tile kernel does not take run the work as a dequant launch of its own
 * after the GEMM. */
typedef struct dk_side_dequant {
  const uint8_t* packed;
  const uint8_t* qabs;
  const float* scale2;
  const float* offset2;
  const float* code2;
  const float* nf4;
  void* out;
  int64_t sb0, sb1;   /* second-level blocks (16384 weights each) */
  int32_t wgs;        /* 1 .. 1024, or DK_SIDE_WGS_AUTO: as many as the CUs the launch's last
                         round of tiles leaves idle (at least 16) */
} dk_side_dequant;
#define DK_SIDE_WGS_AUTO (-1)

/* dk_lora_down_multi and a dequant in one launch: the LoRA downs of `terms` over x, and second-
 * level blocks [side->sb0, side->sb1) of side's layer into side->out as dk_side_dequant describes
 * (side->wgs is not used: one wave per second-level block).  z and the fp16 weights are
 * bit-identical to dk_lora_down_multi's and dk_nf4_dequant's; the two must not overlap in memory.
 * It runs the next layer's dequant ahead of use (k_nf4.dequant_range, solution/k_nf4.py:176-181,
 * issued by solution/fast_qwen.py:729-731) and that layer's q/v LoRA downs
 * (solution/fast_qwen.py:943-944, solution/k_norm.py:49-53) together: no counterpart in the
 * reference as one call.  Terms that mix masked and unmasked inputs, m = 0 or an empty block range
 * run as the separate calls. */
int dk_lora_down_multi_dequant(const void* x, int64_t m, int64_t k, int64_t rank,
                               const dk_lora_down_term* terms, int n_terms,
                               const dk_side_dequant* side, hipStream_t stream);

int64_t dk_h16_workspace(int64_t m, int64_t rows, int64_t cols, int op);
int dk_h16_linear_fwd_lora(const void* x, int64_t ldx, int64_t m, const void* w16, int64_t rows,
                           int64_t cols, const void* bias, const dk_lora_term* terms, int n_terms,
                           int64_t rank, void* y, int64_t ldy, void* workspace,
                           int64_t workspace_bytes, const dk_side_dequant* side,
                           hipStream_t stream);
/* The fused QKV projection with the QKV epilogue's forward folded into the GEMM epilogue:
 * dk_h16_linear_fwd_lora's y, but the output columns [0, rope->cols) (the q and k heads, head size
 * rope->hd = 128) rotated by [x1 c - x2 s | x2 c + x1 s], c, s = cos/sin_table[pos[row] * hd + j],
 * j < hd / 2, from the fp32 sum fp32(fp16(x W^T + bias)) + s fp32(fp16(z B^T)) before the single
 * fp16 rounding — the order of qkv_epilogue_fwd_kernel (solution/k_rope.py:23-61) on the
 * reference's q16 and lq16 (solution/fast_qwen.py:943-949).  Columns past rope->cols (the v
 * heads) are dk_h16_linear_fwd_lora's.  Runs on the 256 x 256-tile kernel only (output columns a
 * multiple of 256, K of 64): DK_ERR_INVALID for other shapes.  pos int32 [m]; tables fp32
 * [positions, hd], 16-byte aligned. */
typedef struct dk_rope {
  const int32_t* pos;
  const float* cos_table;
  const float* sin_table;
  int32_t hd;
  int64_t cols;
} dk_rope;
int dk_h16_linear_fwd_rope(const void* x, int64_t ldx, int64_t m, const void* w16, int64_t rows,
                           int64_t cols, const void* bias, const dk_lora_term* terms, int n_terms,
                           int64_t rank, const dk_rope* rope, void* y, int64_t ldy,
                           const dk_side_dequant* side, hipStream_t stream);
int dk_h16_linear_bwd_dx_lora(const void* dy, int64_t lddy, int64_t m, const void* w16,
                              int64_t rows, int64_t cols, const dk_lora_term* terms, int n_terms,
                              int64_t rank, void* dx, int64_t lddx, int out_mode, void* workspace,
                              int64_t workspace_bytes, const dk_side_dequant* side,
                              hipStream_t stream);
/* dk_h16_linear_bwd_dx_lora that also computes the LoRA column sums `sums` (or NULL: none): the
 * q|k|v backward of a layer after dk_lora_dz_multi (mm(dqkv, W_qkv) with the lq and lv terms,
 * solution/fast_qwen.py:1364, 1376-1380, and the dA and dB of the same terms, 1369, 1371) with
 * one launch fewer.  The sums run on extra workgroups of the GEMM launch, which start on the CUs
 * its tiles leave idle, before `side`'s dequant workgroups; a GEMM that the 256 x 256-tile kernel
 * does not take, or a rank other than 16, runs them as a launch of their own after the GEMM.
 * dA and dB must not overlap anything the GEMM reads or writes. */
int dk_h16_linear_bwd_dx_lora_sums(const void* dy, int64_t lddy, int64_t m, const void* w16,
                                   int64_t rows, int64_t cols, const dk_lora_term* terms,
                                   int n_terms, int64_t rank, void* dx, int64_t lddx, int out_mode,
                                   void* workspace, int64_t workspace_bytes,
                                   const dk_side_dequant* side, const dk_side_lora_sums* sums,
                                   hipStream_t stream);
/* dk_h16_linear_bwd_dx_lora without a workspace argument, allocating nothing.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  The split-K partials go to a
 * library-owned device array of DK_NOALLOC_SCRATCH_BYTES (64 MiB) per device, held until the
 * process ends (every split plan on a 256-CU MI355X fits it); a plan that needs more returns
 * DK_ERR_WORKSPACE before any launch.  Results are bit-identical to dk_h16_linear_bwd_dx_lora
 * with a workspace of dk_h16_workspace bytes.  Every call on a device shares that device's array:
 * calls that overlap on one device (two streams, two threads) race and must be serialised by the
 * caller.  The array's device address is looked up (hipGetSymbolAddress) by the first call on
 * each device; under stream capture that first call returns DK_ERR_CAPTURE before doing anything,
 * so a caller that captures makes one call outside capture first (any later call, captured or
 * not, uses the address found then). */
#define DK_NOALLOC_SCRATCH_BYTES (64ll << 20)
int dk_h16_linear_bwd_dx_lora_noalloc(const void* dy, int64_t lddy, int64_t m, const void* w16,
                                      int64_t rows, int64_t cols, const dk_lora_term* terms,
                                      int n_terms, int64_t rank, void* dx, int64_t lddx,
                                      int out_mode, const dk_side_dequant* side,
                                      hipStream_t stream);
int dk_h16_gateup_swiglu_fwd(const void* x, int64_t ldx, int64_t m, const void* w16, int64_t rows,
                             int64_t cols, void* act, void* gu_out, void* workspace,
                             int64_t workspace_bytes, const dk_side_dequant* side,
                             hipStream_t stream);
int dk_h16_down_swiglu_bwd(const void* dh, int64_t lddh, int64_t m, const void* w16,
                           int64_t rows, int64_t cols, void* gu, void* workspace,
                           int64_t workspace_bytes, const dk_side_dequant* side,
                           hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DK_H */
