/* rlbfp.h: C ABI of the MI355X (gfx950) bfp16-weight GEMM path.
 *
 * Format "bfp16ebs8": a block is 8 consecutive values stored in 9 bytes [E][q0..q7]; value = q_i * 2^(E-133), E =
 * the block's largest float32 exponent field, q_i = clip(rint(x_i * 2^(133-E)), -128, 127), round half to even
 * (redline/npu_layouts.py:62-73, :90-94). Blocks run along K for both GEMM operands.
 *
 * Conventions for every entry point:
 *   - pointers are device pointers (HIP global memory) unless stated; sizes are int64 element counts;
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream); work is enqueued, never synchronised;
 *   - outputs are caller-allocated. No entry point allocates device memory, with one exception: rl_bfp16_gemm and
 *     rl_bfp16_gemm_grouped given an A in a format other than RL_A_BF16 stage it as bf16 in a stream-ordered
 *     allocation (hipMallocAsync / hipFreeAsync on the call's stream; refused under graph capture);
 *   - the return value is RL_OK (0) or an RL_ERR_* code; rl_last_error() gives a message for the calling thread.
 * The reference's interfaces are Python (numpy host code and NPU artifacts run through XRT); each declaration cites
 * the reference function it replaces.
 */
#ifndef RLBFP_H
#define RLBFP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------------------------------------- */
enum {
  RL_OK = 0,
  RL_ERR_NULL = 1,      /* a required pointer is NULL */
  RL_ERR_SHAPE = 2,     /* a size is not a multiple the layout needs, or is out of range */
  RL_ERR_ARG = 3,       /* an enum or flag value is unknown, or arguments contradict each other */
  RL_ERR_ALIGN = 4,     /* a pointer or leading dimension breaks the kernel's alignment */
  RL_ERR_DEVICE = 5,    /* the current device is not gfx950, or a HIP call failed */
  RL_ERR_WORKSPACE = 6  /* the scratch buffer passed in is too small */
};

/* ---- element types ---------------------------------------------------------------------------------------------- */
enum { RL_DTYPE_F32 = 0, RL_DTYPE_BF16 = 1 };

/* ---- block orders of a packed stream ---------------------------------------------------------------------------
 * For an (R, C) matrix with blocks of 8 consecutive columns of a row, unless stated.                              */
enum {
  RL_ORDER_ROWBLOCK = 0, /* row major: block (r, c/8) at index r*(C/8) + c/8, i.e. to_bfp16(x.reshape(-1))          */
  RL_ORDER_A_LAYOUT = 1, /* to_bfp16(a_layout(x, 128, 64)), npu_layouts.py:18-22; R%128 == 0, C%64 == 0             */
  RL_ORDER_B_LAYOUT = 2, /* x is a Linear weight W (N=R rows, K=C cols); to_bfp16(b_layout(W.T, 64, 128)),
                            npu_layouts.py:11-15 and pack_weights.py:72-79; R%128 == 0, C%64 == 0                  */
  RL_ORDER_C_ATB = 3     /* to_bfp16(c_layout_atb(x, 128, 128)), npu_layouts.py:42-47; R%512 == 0, C%1024 == 0      */
};

/* Encode an (rows, cols) row-major matrix (leading dimension ld_x elements) to bfp16, bit-exact to the CPU packer.
 * packed: 9*rows*cols/8 bytes in `order` (may be NULL); deq: the decoded values as bf16, row major rows x cols
 * (may be NULL; the exact bfp16 values, consumed directly by rl_bfp16_gemm with RL_A_BF16). cols % 8 == 0.
 * Replaces npu_layouts.to_bfp16 (redline/npu_layouts.py:62-73) composed with a_layout / b_layout / c_layout_atb
 * (:11-22, :42-47), and pack_weights.pack_b (redline/pack_weights.py:72-79) for order RL_ORDER_B_LAYOUT. */
int rl_bfp16_quantize(const void *x, int32_t x_dtype, int64_t rows, int64_t cols, int64_t ld_x, int32_t order,
                      uint8_t *packed, uint16_t *deq, void *stream);

/* Decode a packed stream in `order` back to an (rows, cols) row-major matrix of out_dtype (exact).
 * Replaces npu_layouts.from_bfp16 (redline/npu_layouts.py:90-94) composed with a_unlayout / b_unlayout /
 * c_unlayout_atb (:56-59, :50-53, :31-39). For RL_ORDER_B_LAYOUT the output is W (N rows, K cols). */
int rl_bfp16_dequantize(const uint8_t *packed, int32_t order, int64_t rows, int64_t cols, void *out,
                        int32_t out_dtype, void *stream);

/* ---- GEMM -------------------------------------------------------------------------------------------------------
 * C = epilogue(A @ B), A (M, K), B (K, N) packed in b_layout(64, 128) order (the bytes pack_weights.py writes),
 * fp32 accumulation on bf16 MFMA, bf16 output. M >= 1, N % 128 == 0, K % 64 == 0.                                  */
enum {
  RL_A_BF16 = 0,          /* bf16 row major, used as is (already bfp16 values, e.g. rl_bfp16_quantize's deq)  */
  RL_A_BF16_QUANTIZE = 1, /* bf16 row major, quantized to bfp16 along K by a staging pass before the product    */
  RL_A_PACKED_ROWBLOCK = 2, /* packed, RL_ORDER_ROWBLOCK of (M, K); lda ignored                                   */
  RL_A_PACKED_A_LAYOUT = 3  /* packed, RL_ORDER_A_LAYOUT of (M, K) (the NPU's A operand); M%128 == 0; lda ignored */
};
enum {
  RL_ACT_NONE = 0,
  RL_ACT_GELU_TANH = 1, /* x * sigmoid(2u), u = sqrt(2/pi)(x + 0.044715 x^3) (kernels/vlm/gelu_bfp.cc:1-8)        */
  RL_ACT_SWIGLU = 2     /* B columns interleaved [gate 64 | proj 64] per 128 (pack_weights.py:82-89): output (M, N/2),
                           out[:, 64t+u] = silu(v[:, 128t+u]) * v[:, 128t+64+u] (kernels/atb3/mm_bfp_swiglu.cc)  */
};
enum {
  RL_EP_QUANTIZE_OUT = 1, /* after the bf16 rounding, re-quantize each 8-column block of the output to bfp16 (the
                             stored bf16 values are then exact bfp16 values, ready as the next GEMM's RL_A_BF16)   */
  RL_EP_WHOLE_K = 2       /* rl_bfp16_gemm_ws: never split K, whatever the workspace; the workspace then needs only
                             the staged bf16 copy of a non-bf16 A (M * K * 2 bytes rounded up to 256), or nothing */
};

/* Layout of the bf16 C. */
enum {
  RL_C_ROWMAJOR = 0, /* (M, Nout) row major, leading dimension ldc */
  RL_C_ATB = 1       /* flat, the c_layout_atb(., 128, 128) element order (npu_layouts.py:42-47), i.e. the C16
                        artifacts' output (kernels/vlm/mm_bfp_c16.cc:1-2); M % 512 == 0, Nout % 1024 == 0; ldc ignored */
};

/* Fused epilogue, applied in fp32 in this order: v = acc + bias[n]; v = act(v); v = residual[m][n] + g[n] * v with
 * g = gate row 1 for rows < gate_split_row else gate row 0 (gate NULL = 1); out = bf16(v) (RNE); optional
 * re-quantize. The gate/residual step is the adaLN "x' = x + g * branch" (redline/run_ln.py:65-67, rows_param
 * :82-86; kernels/glue/ln_mod.cc:92-143) fused into the producing GEMM. n indexes output columns.
 * packed_out (optional) receives to_bfp16 of the bf16 output (blocks of 8 output columns of a row) in packed_order,
 * written by the GEMM's own epilogue: RL_ORDER_C_ATB, the reference GEMM's bfp16 C stream (M % 512 == 0, Nout %
 * 1024 == 0; kernels/atb3/mm_bfp_mixed.cc:153-168), or RL_ORDER_A_LAYOUT, the next GEMM's A operand as the SwiGLU GEMM
 * pushes H (M % 128 == 0, Nout % 64 == 0; kernels/atb3/mm_bfp_swiglu.cc:73-86). With packed_out, C may be NULL;
 * otherwise C also receives the bf16 values (re-quantized with RL_EP_QUANTIZE_OUT, so they equal the packed blocks). */
typedef struct rl_epilogue {
  int32_t act;               /* RL_ACT_* */
  int32_t flags;             /* RL_EP_* */
  const float *bias;         /* [N] (pre-activation, all computed columns) or NULL */
  const float *gate;         /* [Nout] or [2][Nout] (row 1 used for rows < gate_split_row) or NULL */
  int64_t gate_split_row;    /* 0 = every row uses gate row 0 */
  const uint16_t *residual;  /* bf16 (M, Nout) with leading dimension ld_residual, or NULL */
  int64_t ld_residual;
  uint8_t *packed_out;       /* 9 * M * Nout / 8 bytes, 4-byte aligned, or NULL */
  int32_t packed_order;      /* RL_ORDER_C_ATB or RL_ORDER_A_LAYOUT (when packed_out is set) */
  int32_t c_order;           /* RL_C_ROWMAJOR or RL_C_ATB */
} rl_epilogue;

/* One GEMM. lda / ldc in elements (bf16); ldc >= Nout (N, or N/2 for SwiGLU). ep may be NULL (plain bf16 C).
 * An A format other than RL_A_BF16 is staged as bf16 first (see rl_bfp16_gemm_ws) in a stream-ordered allocation
 * (hipMallocAsync / hipFreeAsync on `stream`); on a stream under graph capture that is refused with
 * RL_ERR_WORKSPACE, and rl_bfp16_gemm_ws with a workspace or rl_bfp16_gemm_noalloc serves instead.
 * Replaces forward.gemm / NPU.run(op, GEMMS[op, M], [A, B, C]) (redline/forward.py:194-197, :138-165), the ATB
 * microkernels matmul_vectorized_bfp16 (kernels/atb3/mm_bfp_mixed.cc:61, mm_bfp_rho.cc:64, vlm/mm_bfp_c16.cc:62)
 * and, with RL_ACT_SWIGLU, matmul_swiglu_bfp16 (kernels/atb3/mm_bfp_swiglu.cc:88). */
int rl_bfp16_gemm(const void *A, int32_t a_fmt, int64_t lda, const uint8_t *B_packed, uint16_t *C, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, const rl_epilogue *ep, void *stream);

/* rl_bfp16_gemm with a caller's workspace (device memory, 16-byte aligned). It serves two purposes:
 *   - a GEMM whose output tiles fill few compute units (small M, deep K: the text encoder's down projection at
 *     M = 512, K = 12288) may split K into pieces that run side by side. Each piece writes fp32 partial sums to the
 *     workspace; a second launch adds them in piece order and applies the epilogue as above (results differ from
 *     the whole-K sums by fp32 rounding only);
 *   - an A in any format other than RL_A_BF16 (the NPU's packed A layout above all: every GEMM of
 *     redline/forward.py passes A that way, :32, :245) is first staged as bf16 in the workspace (its exact bfp16
 *     values, one HBM-bound pass: 9/8 + 2 bytes per value), and the product then runs on the RL_A_BF16 kernel with
 *     the rest of the workspace. The result is the RL_A_BF16 path's on the staged values: bit-identical to
 *     rl_bfp16_gemm's for the same format unless the K split applies.
 * workspace NULL: exactly rl_bfp16_gemm, which runs every shape and A format whole K (a non-bf16 A then stages into
 * a stream-ordered allocation that holds the staged copy only, M * K * 2 bytes rounded up to 256).
 * A workspace below rl_bfp16_gemm_workspace_size() for the shape and format (below the staged copy alone with
 * RL_EP_WHOLE_K) returns RL_ERR_WORKSPACE before anything is enqueued (nothing is written to the workspace or C). Calls that share a workspace on different streams race.
 * Same reference interface as rl_bfp16_gemm (redline/forward.py:194-197). */
int rl_bfp16_gemm_ws(const void *A, int32_t a_fmt, int64_t lda, const uint8_t *B_packed, uint16_t *C, int64_t ldc,
                     int64_t M, int64_t N, int64_t K, const rl_epilogue *ep, void *workspace, int64_t workspace_bytes,
                     void *stream);
/* Workspace bytes rl_bfp16_gemm_ws needs for an RL_A_BF16 GEMM of this shape on the current device (0: this shape
 * runs whole; -1: the shape is invalid). */
int64_t rl_bfp16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);
/* Workspace bytes rl_bfp16_gemm_ws uses for this A format and shape: the staged bf16 A for a non-bf16 format
 * (M * K * 2 rounded up to 256), plus the K-split partials; -1: invalid shape or format. */
int64_t rl_bfp16_gemm_workspace_size(int32_t a_fmt, int64_t M, int64_t N, int64_t K);

/* rl_bfp16_gemm_ws without a workspace argument and without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart
 * in the reference. The workspace is a fixed device array of RL_NOALLOC_SCRATCH_BYTES inside the library; each GPU
 * the library runs on holds its own copy until the process ends. Shapes and A formats whose
 * rl_bfp16_gemm_workspace_size() exceeds it are rejected with RL_ERR_WORKSPACE (64 MiB holds, e.g., the K-split
 * partials of the text encoder's down projection at M = 512 and the staged A of up to 32M values). Results are those
 * of rl_bfp16_gemm_ws with a workspace of that size. Every call on one GPU shares that GPU's array, and no byte of it
 * is read before the same call wrote it: calls that overlap on one GPU (different streams or threads) race. */
#define RL_NOALLOC_SCRATCH_BYTES (64ll << 20)
int rl_bfp16_gemm_noalloc(const void *A, int32_t a_fmt, int64_t lda, const uint8_t *B_packed, uint16_t *C, int64_t ldc,
                          int64_t M, int64_t N, int64_t K, const rl_epilogue *ep, void *stream);

/* Several independent GEMMs (different shapes, weights and epilogues, one A format) in one launch, e.g. the image-
 * and text-stream projections of a DiT block. At most RL_MAX_GROUP descriptors. A non-bf16 A format stages every
 * member's A as bf16 first, in one stream-ordered allocation (as rl_bfp16_gemm does). Replaces the per-op sequence of
 * CachedStep.blocks (redline/forward.py:240-254) for GEMMs that do not depend on each other. */
#define RL_MAX_GROUP 16
typedef struct rl_gemm_desc {
  const void *A;
  int64_t lda;
  const uint8_t *B_packed;
  uint16_t *C;
  int64_t ldc;
  int64_t M, N, K;
  rl_epilogue ep;
} rl_gemm_desc;
int rl_bfp16_gemm_grouped(const rl_gemm_desc *descs, int32_t n, int32_t a_fmt, void *stream);

/* ---- GEMV (adaLN modulation) -------------------------------------------------------------------------------------
 * y (M, N) bf16 = Q(act(x)) @ B, x (M, K) bf16 with leading dimension ldx, B packed in b_layout(64, 128) order,
 * 1 <= M <= 8, N % 128 == 0, K % 64 == 0; act = RL_ACT_NONE or RL_GEMV_SILU (evaluated in fp32); Q quantizes the
 * activation to bfp16 blocks of 8 along K as the GEMM's A operand is, so every block product is exact in int32;
 * fp32 accumulation, bf16 output. Replaces host_glue.modulation / linear(silu(te), W) (redline/host_glue.py:22-28,
 * :43-48), which the reference runs in numpy float32 on the host. */
enum { RL_GEMV_SILU = 3 };
int rl_bfp16_gemv(const uint16_t *x, int64_t ldx, const uint8_t *B_packed, uint16_t *y, int64_t ldy, int64_t M,
                  int64_t N, int64_t K, int32_t act, void *stream);

/* ---- residual add + LayerNorm / RMSNorm + modulate -> the next GEMM's A ----------------------------------------
 * For each row r of (M, D):
 *   x'[r] = bf16(x[r] + g * branch[r])   one fp32 fma, then RNE; branch NULL means 0;
 *   y[r]  = (x'[r] - mean) * rstd * sc   fp32; RL_NORM_LAYER: mean and variance of the row's D values of x' (eps
 *                                        1e-6, no affine); RL_NORM_RMS: mean = 0, rstd = 1 / sqrt(mean(x'^2) + 1e-6);
 * then y is quantized to bfp16 blocks of 8 along the row (as rl_bfp16_quantize does).
 * g and sc come from params, (2, 2D) bf16 with row p = [g (D) | sc (D)] (run_ln.ln_params, redline/run_ln.py:38-40;
 * vlm_run.rms_params, redline/vlm_run.py:62-65). Rows r < split_row use params row 1, the rest row 0
 * (run_ln.rows_param, redline/run_ln.py:82-86; the reference's S is split_row / 128).
 * The branch is bf16 row major (ld_br), or bfp16 packed in RL_ORDER_ROWBLOCK of (M, D) (ld_br ignored).
 * Outputs (each may be NULL, not all three):
 *   x_out: x' as bf16 row major (ld_xo); may equal x;
 *   a_packed: 9*M*D/8 bytes of y in a_order (RL_ORDER_ROWBLOCK, or RL_ORDER_A_LAYOUT with M % 128 == 0);
 *   a_deq: y's bfp16 values as bf16, row major (ld_a), the next rl_bfp16_gemm's RL_A_BF16 operand.
 * D % 64 == 0 and 64 <= D <= 8192.
 * Replaces the fused residual + LayerNorm + modulate artifact, kernels/glue/ln_design.py:38-118 with ln_mod.cc:92-204,
 * run by run_ln.ln_run (redline/run_ln.py:43-57). With RL_NORM_RMS it replaces its RMSNorm copies
 * (kernels/vlm/rms_mod.cc, rms16_mod.cc for a bf16 branch) run by LM._rms (redline/vlm_run.py:343-344). */
enum { RL_NORM_LAYER = 0, RL_NORM_RMS = 1 };
enum { RL_BRANCH_BF16 = 0, RL_BRANCH_PACKED = 1 };
int rl_ln_modulate(const uint16_t *x, int64_t ldx, const void *branch, int32_t br_fmt, int64_t ld_br,
                   const uint16_t *params, int64_t split_row, int32_t norm, uint16_t *x_out, int64_t ld_xo,
                   uint8_t *a_packed, int32_t a_order, uint16_t *a_deq, int64_t ld_a, int64_t M, int64_t D,
                   void *stream);

/* ---- QKV post: the QKV GEMM output -> attention Q / K / V --------------------------------------------------------
 * C (M, 3 * heads * 128) bf16 row major (ldc): per token row the q, k and v columns of `heads` heads of 128 dims.
 * Per head and token row, in fp32:
 *   Q = rope(rms(q) * wq), K = rope(rms(k) * wk), V = v,
 * with rms(x) = x / sqrt(mean(x^2) + 1e-6) over the head's 128 dims, and rope the rotation of each dim pair
 * (2i, 2i+1) by (cos, sin)[row][i] (run_glue.rms_rope / rope, redline/run_glue.py:27-37). Q and K are quantized to
 * bfp16 in blocks of 8 dims, V in blocks of 8 tokens of one dim.
 * cos, sin: (M, 64) bf16 each, row major; wq (the attention score scale log2(e)/sqrt(128) folded in, as
 * redline/run_qkv.py:27 does) and wk: 128 bf16 each.
 * Outputs (each may be NULL, not all):
 *   q_tiles  (heads, M/64, 9216 bytes): per head and 64-token tile, to_bfp16(a_layout(Q tile, 64, 128));
 *   kv_tiles (heads, M/64, 2, 9216 bytes): to_bfp16(b_layout(K tile^T, 128, 64)), then to_bfp16(b_layout(V tile, 64,
 *            128)) (the attention kernel's formats, kernels/glue/qkv_post.cc:1-16);
 *   q, k     (heads, M, 128) bf16 each: the same quantized values, head major;
 *   v        (heads, 128, M) bf16: V transposed (V^T per head, token columns), the layout rl_attention reads.
 * M % 64 == 0, heads >= 1.
 * Replaces the QKV-post artifact (kernels/glue/qkv_design.py:40-118 with qkv_post.cc:134-177) run by
 * run_qkv.qkv32_npu (redline/run_qkv.py:67-82). */
int rl_qkv_post(const uint16_t *C, int64_t ldc, int64_t M, int32_t heads, const uint16_t *cos, const uint16_t *sin,
                const uint16_t *wq, const uint16_t *wk, uint8_t *q_tiles, uint8_t *kv_tiles, uint16_t *q, uint16_t *k,
                uint16_t *v, void *stream);

/* rl_qkv_post for grouped-query attention: C (M, (hq + 2 hkv) * 128) holds per token row the q columns of hq heads,
 * then the k and v columns of hkv heads each. Outputs as above with hq Q heads and hkv K / V heads: q_tiles (hq, M/64,
 * 9216), kv_tiles (hkv, M/64, 2, 9216), q (hq, M, 128), k (hkv, M, 128), v (hkv, 128, M). hq == hkv is rl_qkv_post.
 * Replaces the text encoder's GQA QKV-post artifacts (kernels/vlm/qkv_gqa_design.py, 32 q and 8 kv heads, with the
 * same microkernels kernels/glue/qkv_post.cc) run by LM._layer (redline/vlm_run.py:433-437). */
int rl_qkv_post_gqa(const uint16_t *C, int64_t ldc, int64_t M, int32_t hq, int32_t hkv, const uint16_t *cos,
                    const uint16_t *sin, const uint16_t *wq, const uint16_t *wk, uint8_t *q_tiles, uint8_t *kv_tiles,
                    uint16_t *q, uint16_t *k, uint16_t *v, void *stream);

/* ---- attention over the QKV post pass's output -------------------------------------------------------------------
 * Per head h and query i: O[i][(h0 + h) * 128 + d] = sum_j P[i][j] V[j][d], P = 2^(S - max) / sum over the visible
 * keys, S = Q K^T. Q carries the score scale log2(e)/sqrt(128) (as rl_qkv_post's wq does), so S is in log2 units.
 * Key j is visible to query i when j < nkv and, with lim, j <= lim[i].
 * Arithmetic: fp32 scores, running max and sums; P rounded to bf16 for the second product; fp32 accumulation; bf16
 * out. With quantize_out, each 8-dim block of O is quantized to bfp16, making O the out-projection GEMM's RL_A_BF16
 * operand.
 * q (heads, nq, 128), k (heads, nk, 128), vt (heads, 128, nk) = V transposed: rl_qkv_post's native outputs, bf16.
 * o: row major with leading dimension ldo, head h at columns (h0 + h) * 128. lim: nq int32 or NULL.
 * nq % 128 == 0, nk % 64 == 0, 1 <= nkv <= nk.
 * Replaces the attention artifacts (kernels/attn/attn_bfp.cc with attn_design.py) run by run_attn.attn_npu
 * (redline/run_attn.py:67-82) and NPU.run("attn", ...) (redline/forward.py:247, :369-377). */
int rl_attention(const uint16_t *q, const uint16_t *k, const uint16_t *vt, int32_t heads, int64_t nq, int64_t nk,
                 int64_t nkv, const int32_t *lim, uint16_t *o, int64_t ldo, int32_t h0, int32_t quantize_out,
                 void *stream);

/* rl_attention with a caller's workspace (device memory, 16-byte aligned), which lets the launch split work along the
 * keys: the tasks (head, 128-query block) that fill whole rounds of the GPU's resident workgroups run whole, and when
 * the tasks left over fill at most 4/5 of a round their key blocks are spread over every resident workgroup. A task
 * cut into pieces leaves fp32 partials (unnormalised O, running max, sum) in the workspace, merged in piece order by
 * a second launch on the same stream (the result does not depend on timing). Same arguments and results as
 * rl_attention; summation order differs from the unsplit launch within fp32 rounding.
 * workspace NULL: every task runs whole. workspace_bytes below rl_attention_workspace_bytes(): RL_ERR_WORKSPACE.
 * Calls that share a workspace on different streams race. Same reference interface as rl_attention. */
int rl_attention_ws(const uint16_t *q, const uint16_t *k, const uint16_t *vt, int32_t heads, int64_t nq, int64_t nk,
                    int64_t nkv, const int32_t *lim, uint16_t *o, int64_t ldo, int32_t h0, int32_t quantize_out,
                    void *workspace, int64_t workspace_bytes, void *stream);
/* Workspace bytes rl_attention_ws needs for this shape on the current device (0: no split for this shape; -1: the
 * shape is invalid). Without a usable device the plan assumes 256 compute units. */
int64_t rl_attention_workspace_bytes(int32_t heads, int64_t nq, int64_t nk);

/* ---- host-only helpers (no GPU needed) ---------------------------------------------------------------------------- */
/* Shape/argument checks the entry points run before launching, callable on a machine without a GPU. */
int rl_validate_ln(int64_t ldx, int32_t br_fmt, int64_t ld_br, int32_t norm, int64_t ld_xo, int32_t a_order,
                   int64_t ld_a, int64_t split_row, int64_t M, int64_t D);
int rl_validate_qkv_post(int64_t ldc, int64_t M, int32_t heads);
int rl_validate_qkv_post_gqa(int64_t ldc, int64_t M, int32_t hq, int32_t hkv);
int rl_validate_attention(int32_t heads, int64_t nq, int64_t nk, int64_t nkv, int64_t ldo, int32_t h0);
int rl_validate_quantize(int32_t x_dtype, int64_t rows, int64_t cols, int64_t ld_x, int32_t order);
int rl_validate_gemm(int32_t a_fmt, int64_t lda, int64_t ldc, int64_t M, int64_t N, int64_t K, const rl_epilogue *ep);
int rl_validate_gemv(int64_t ldx, int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t act);
/* Bytes of a packed stream holding rows x cols values (9 per 8). */
int64_t rl_packed_bytes(int64_t rows, int64_t cols);
/* Message for the last error on the calling thread ("" after success). */
const char *rl_last_error(void);
/* Library version string. */
const char *rl_version(void);
/* RL_OK when the current HIP device is a gfx950 (MI355X); RL_ERR_DEVICE otherwise. Initialises HIP. */
int rl_device_check(void);

#ifdef __cplusplus
}
#endif

#endif /* RLBFP_H */
