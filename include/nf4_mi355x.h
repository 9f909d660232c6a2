/*
 * nf4_mi355x.h - C ABI of the MI355X (gfx950) NF4 quantized-linear library.
 *
 * The library dequantizes bitsandbytes-layout NF4 weights and multiplies with them, forward and
 * backward, on one AMD Instinct MI355X.  Every entry point takes plain device pointers, sizes, a
 * dtype code and a HIP stream (as void*), launches asynchronously on that stream and returns an
 * int status (NF4_OK == 0).  The caller allocates every output and workspace, and apart from
 * one entry point the library owns no device memory and keeps no state between calls, so it is
 * reentrant and thread-safe.  The exception is nf4_linear_dx_noalloc (for callers that cannot
 * allocate): its split-K partials live in a 64 MiB device array that the library holds on every
 * GPU it runs on until the process ends, and calls of it that overlap on one GPU race.
 *
 * Weight format (bitsandbytes 0.50.2 QuantState, as read by the reference at
 * /root/reference/solution/nf4.py:46-53,112-131):
 *   packed   uint8 [ceil(rows*cols/2)]: element i of the row-major weight in byte i/2,
 *            high nibble for even i (nf4.py:33-35);
 *   absmax   per block of `blocksize` elements: uint8 codes when nested (double quant),
 *            fp32 otherwise;
 *   absmax2  fp32 [ceil(nblocks/blocksize2)] and code2 fp32[256] (nested only);
 *   offset   fp32 mean added after the 8-bit dequant (nested only);
 *   code     fp32[16], the NF4 table.
 * Dequantized element: round(code[nib] * (fp32(code2[q] * absmax2[b / blocksize2]) + offset))
 * with every product/sum rounded separately in fp32 and one round-to-nearest-even at the end.
 */
#ifndef NF4_MI355X_H
#define NF4_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NF4_ABI_VERSION 4

/* status codes */
#define NF4_OK 0
#define NF4_ERR_ARG 1          /* null pointer, negative size, bad dtype, misaligned pointer */
#define NF4_ERR_UNSUPPORTED 2  /* a layout or shape this library does not cover */
#define NF4_ERR_LAUNCH 3       /* the HIP runtime reported an error */
#define NF4_ERR_WORKSPACE 4    /* the workspace passed is smaller than required */

/* dtype codes: activations, outputs and (for dequant) the dequantized weight */
#define NF4_F16 0
#define NF4_BF16 1
#define NF4_F32 2
#define NF4_I32 3  /* int32 sums (nf4_int8_gemm output only) */

/* One NF4 weight [rows, cols] (out_features x in_features) in bitsandbytes layout. */
typedef struct nf4_weight {
    const uint8_t *packed;
    const void *absmax;    /* uint8 [nblocks] if nested else fp32 [nblocks] */
    const float *absmax2;  /* nested: fp32 [ceil(nblocks / blocksize2)], else NULL */
    const float *code2;    /* nested: fp32 [256], else NULL */
    const float *code;     /* fp32 [16] */
    float offset;          /* nested: the mean offset, else 0 */
    int32_t nested;
    int64_t rows;
    int64_t cols;
    int32_t blocksize;
    int32_t blocksize2;
} nf4_weight;

/* A rank-r LoRA adapter on output segment `seg` of a stacked projection (peft semantics,
 * y_seg += scale * drop(x) @ A^T @ B^T; reference layer.py:875-878, 1072-1090).
 * Forward reads t and b.  With a == NULL, t holds drop(x) @ A^T (the caller's nf4_lora_xa).
 * With a set (dropout off: drop(x) = x), the forward computes t = x @ A^T itself, rounded to
 * the GEMM dtype as nf4_lora_xa rounds it, writes it to t (then a writable [M, rank] buffer:
 * the backward pass needs it) and uses it; on the skinny small-M path (3 to 32 tokens, rank
 * <= 16) inside the GEMM's own launch, else in a launch of its own before the GEMM.
 * The input-gradient GEMM reads a and da. */
typedef struct nf4_lora {
    int32_t seg;
    int32_t rank;          /* 1..64 */
    float scale;           /* alpha / r */
    const void *t;         /* [M, rank] drop(x) @ A^T, GEMM dtype (forward; written if a) */
    const void *b;         /* [rows_seg, rank] LoRA B, GEMM dtype (forward) */
    const void *a;         /* [rank, K] LoRA A, GEMM dtype (input gradient; forward: see
                            * above), 16-byte aligned in the forward */
    const void *da;        /* [M, rank] scale * dY_seg @ B, GEMM dtype (input gradient) */
} nf4_lora;

/* Library version / status text. */
int nf4_abi_version(void);
const char *nf4_status_string(int status);

/* ---------------------------------------------------------------- standalone dequantization */

/* out[rows, cols] = dequant(w) in out_dtype (F16, BF16 or F32).
 * Replaces: dequantize_nf4(packed, quant_state, dtype) -> nf4_dequant_kernel
 *           (/root/reference/solution/nf4.py:26-38, 69-77), with the absmax rebuild of
 *           _absmax_fp32 (nf4.py:41-55) folded into the kernel. */
int nf4_dequant(const nf4_weight *w, void *out, int out_dtype, void *stream);

/* Up to NF4_MAX_SEGMENTS weights with equal cols, dequantized one after the other into one
 * stacked [sum(rows), cols] buffer (q|k|v or gate|up).
 * Replaces: _dequant(layers, dtype) -> nf4_dequant_multi_kernel
 *           (/root/reference/solution/layer.py:45-73, 463-493). */
#define NF4_MAX_SEGMENTS 8
int nf4_dequant_multi(const nf4_weight *ws, int nw, void *out, int out_dtype, void *stream);

/* Up to NF4_MAX_SEGMENTS weights of any shapes in one launch, weight i into its own
 * [rows_i, cols_i] buffer outs[i] (e.g. all seven projections of a decoder layer).
 * Replaces: the reference's per-layer sequence of _dequant / dequantize_nf4 calls, one kernel
 *           launch per call (/root/reference/solution/layer.py:463-493; nf4.py:69-77). */
int nf4_dequant_batch(const nf4_weight *ws, int nw, void *const *outs, int out_dtype,
                      void *stream);

/* Any number of weights dequantized by ONE launch through a descriptor table (e.g. all 196
 * projections of a 28-layer model).  The weights are frozen, so the table is built once:
 * nf4_dequant_table_pack validates every weight (fast layout: power-of-two blocksize >= 8,
 * 4-byte aligned packed bytes, 16-byte aligned outputs, < 2^32 elements each; else
 * NF4_ERR_UNSUPPORTED) and writes the table into HOST memory of nf4_dequant_table_bytes()
 * bytes, with the launch's workgroup count in *blocks.  The caller copies the table to device
 * memory (64-byte aligned) once; nf4_dequant_table then launches on that copy with the same nw
 * and blocks, any number of times, writing weight i into outs[i] as nf4_dequant_batch would.
 * The kernel checks the table's tag, dtype, weight and workgroup counts and writes nothing
 * when they do not match the launch.
 * Replaces: a sequence of dequantize_nf4 / _dequant calls, one launch per call
 *           (/root/reference/solution/nf4.py:69-77; layer.py:463-493). */
size_t nf4_dequant_table_bytes(const nf4_weight *ws, int nw);
int nf4_dequant_table_pack(const nf4_weight *ws, int nw, void *const *outs, int out_dtype,
                           void *host_table, size_t table_bytes, int64_t *blocks);
int nf4_dequant_table(const void *dev_table, int nw, int64_t blocks, int out_dtype,
                      void *stream);

/* ------------------------------------------------------------------ fused dequant-GEMMs */

/* Y[M, sum(rows)] = X[M, K] @ W_stack^T (+ bias) (+ sum over loras scale * T @ B^T on the
 * lora's segment columns), W dequantized inside the GEMM main loop, fp32 accumulation, one
 * rounding to dtype (F16 or BF16).  X rows are ldx elements apart, Y rows ldy.
 * Weight: from 3 tokens on, each element is round(code * absmax) in dtype, the dequantized
 * weight bit for bit.  At M <= 2 (the decode GEMV regime, where the reference defers to
 * bitsandbytes' GEMV: fp32 code * fp32 absmax, nf4.py:15-16, 105-118) the product is
 * round(code) * x in fp32, scaled per block by the fp32 absmax: bitsandbytes' arithmetic with
 * the 16 codes rounded to dtype (relative error <= 2^-9 in bf16, 2^-12 in fp16 per code).
 * Replaces: F.linear(x, dequantize_nf4(W), bias) in NF4Linear.forward (nf4.py:84-91); the
 *           addmm / mm projection GEMMs of FusedDecoderLayer.forward with the LoRA terms
 *           (layer.py:871-878, 893, 914, 929); RecomputedMLP's forward GEMMs (mlp.py:47-54).
 * workspace may be NULL when nf4_linear_fwd_workspace() returns 0 for the same arguments. */
int nf4_linear_fwd(const void *x, int64_t m, int64_t ldx,
                   const nf4_weight *ws, int nw, const void *bias,
                   const nf4_lora *loras, int nlora,
                   void *y, int64_t ldy, int dtype,
                   void *workspace, size_t workspace_bytes, void *stream);
size_t nf4_linear_fwd_workspace(int64_t m, const nf4_weight *ws, int nw, int dtype);

/* dX[M, K] (+)= dY[M, sum(rows)] @ W_stack (+ sum over loras da @ A), the transposed
 * dequant-GEMM.  accumulate != 0 adds into dX.
 * Replaces: torch.matmul(grad, dequantize_nf4(W)) in NF4Linear.backward (nf4.py:93-99); the
 *           input-gradient GEMMs of FusedDecoderLayer.backward (layer.py:1015, 1024-1032, 1061,
 *           1086-1088) and RecomputedMLP.backward (mlp.py:65, 72-73). */
int nf4_linear_dx(const void *dy, int64_t m, int64_t lddy,
                  const nf4_weight *ws, int nw,
                  const nf4_lora *loras, int nlora,
                  void *dx, int64_t lddx, int accumulate, int dtype,
                  void *workspace, size_t workspace_bytes, void *stream);
size_t nf4_linear_dx_workspace(int64_t m, const nf4_weight *ws, int nw, int dtype);

/* nf4_linear_dx without a workspace argument: it allocates nothing, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).  No counterpart in the reference.  Split-K partials go to one static
 * device array of NF4_STATIC_SCRATCH_BYTES per GPU, set up when the library's code loads on a
 * device and held until the process ends; its address is looked up on the first call on each
 * device (make that first call outside graph capture).  The tiling is nf4_linear_dx's, chosen
 * among the plans whose partials fit the array (plans with no split need none), so every size
 * is accepted; the result equals nf4_linear_dx's bit for bit whenever its plan fits.  The
 * array keeps the last call's partials; calls that overlap on one GPU (other streams or
 * threads) share it and race.  The stream must belong to the current device. */
#define NF4_STATIC_SCRATCH_BYTES (64u << 20)
int nf4_linear_dx_noalloc(const void *dy, int64_t m, int64_t lddy,
                          const nf4_weight *ws, int nw,
                          const nf4_lora *loras, int nlora,
                          void *dx, int64_t lddx, int accumulate, int dtype, void *stream);

/* The same two GEMMs with the tiling pinned instead of chosen by the library's cost model:
 * tile NF4_TILE_256 (256x256 tiles, 8 waves), NF4_TILE_128 (128x128, 4 waves) or
 * NF4_TILE_128_KSPLIT2 (128x128, two groups of 4 waves splitting each tile's reduction), with
 * every tile's reduction further split `splits` ways across workgroups (1 = none; 2..16, no
 * split may be empty, else NF4_ERR_ARG).  NF4_TILE_AUTO (or any negative tile) is the plain
 * entry point.  A pinned tiling never takes the small-M kernels.  A workspace of
 * splits * M * (output columns) * 4 bytes always suffices.  For callers that autotune or that
 * need one fixed summation order across token counts, and for tests of every tiling.
 * Replaces: the same reference GEMMs as nf4_linear_fwd / nf4_linear_dx (the reference leaves
 *           the tiling to cuBLAS). */
#define NF4_TILE_AUTO (-1)
#define NF4_TILE_256 0
#define NF4_TILE_128 1
#define NF4_TILE_128_KSPLIT2 3
int nf4_linear_fwd_tiled(const void *x, int64_t m, int64_t ldx,
                         const nf4_weight *ws, int nw, const void *bias,
                         const nf4_lora *loras, int nlora,
                         void *y, int64_t ldy, int dtype,
                         void *workspace, size_t workspace_bytes, void *stream,
                         int tile, int splits);
int nf4_linear_dx_tiled(const void *dy, int64_t m, int64_t lddy,
                        const nf4_weight *ws, int nw,
                        const nf4_lora *loras, int nlora,
                        void *dx, int64_t lddx, int accumulate, int dtype,
                        void *workspace, size_t workspace_bytes, void *stream,
                        int tile, int splits);

/* ---------------------------------------------------------------------- LoRA side GEMMs */

/* t[M, rank] = xd[M, K] @ A[rank, K]^T  (LoRA down-projection; layer.py:875, 877). */
int nf4_lora_xa(const void *xd, int64_t m, int64_t k, int64_t ldx, const void *a, int rank,
                void *t, int dtype, void *stream);

/* da[M, rank] = scale * dY[M, N] @ B[N, rank]  (layer.py:1074-1078). */
int nf4_lora_da(const void *dy, int64_t m, int64_t n, int64_t lddy, const void *b, int rank,
                float scale, void *da, int dtype, void *stream);

/* out = scale * U[M, P]^T @ V[M, rank], fp32, reduced over M (the LoRA weight gradients):
 * transpose_out == 0 -> out[P, rank] (dB = s * dY^T @ T, layer.py:1075-1076);
 * transpose_out != 0 -> out[rank, P] (dA = da^T @ xd, layer.py:1080-1081).
 * workspace: nf4_lora_wgrad_workspace() bytes for the split-M partial sums (unused when the
 * one-launch path of nf4_lora_wgrad_multi below applies). */
int nf4_lora_wgrad(const void *u, int64_t m, int64_t p, int64_t ldu, const void *v, int rank,
                   float scale, float *out, int transpose_out, int dtype,
                   void *workspace, size_t workspace_bytes, void *stream);
size_t nf4_lora_wgrad_workspace(int64_t m, int64_t p, int rank);

/* Several LoRA side products in one launch (q and v adapters of a layer).  A job names the
 * rows of its [M, cols] operand (already at the job's first column: da and dB read column
 * ranges of the stacked q|k|v gradient), the small operand and the output. */
#define NF4_MAX_LORA_JOBS 4
typedef struct nf4_lora_job {
    const void *in;        /* [M, cols] operand rows, `ld` elements apart */
    int64_t ld;
    int64_t cols;          /* xa: K; da: N; wgrad: P */
    const void *w;         /* xa: A [rank, cols]; da: B [cols, rank]; wgrad: V [M, rank] */
    void *out;             /* xa / da: [M, rank] GEMM dtype; wgrad: fp32 [cols, rank] or
                            * [rank, cols] (transpose_out) */
    float scale;
    int32_t transpose_out; /* wgrad only */
} nf4_lora_job;

/* t_j = in_j @ A_j^T for every job (nf4_lora_xa per job: layer.py:875, 877). */
int nf4_lora_xa_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, int dtype,
                      void *stream);
/* out_j = scale_j * in_j @ A_j for every job, the LoRA term of the input gradient on its own:
 * in_j = da [M, rank] (row stride ld >= rank), w_j = A [rank, cols], out_j [M, cols]
 * contiguous in the GEMM dtype, fp32 sums rounded once.  For a LoRA input that is not the
 * projection's input x (dropout p > 0), whose gradient the norm backward masks
 * (nf4_rmsnorm_bwd's dq / dv).
 * Replaces: dd_q = da_q @ A_q, dd_v = da_v @ A_v (/root/reference/solution/layer.py:1086-1087). */
int nf4_lora_ax_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, int dtype,
                      void *stream);
/* da_j = scale_j * in_j @ B_j for every job (nf4_lora_da per job: layer.py:1074-1078). */
int nf4_lora_da_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, int dtype,
                      void *stream);
/* out_j = scale_j * in_j^T @ V_j for every job (nf4_lora_wgrad per job: layer.py:1075-1076,
 * 1080-1081): one launch over M when every job's rows load as 16-byte pieces (16-byte aligned
 * `in` with ld % 8 == 0, 16-byte aligned V, rank % 8 == 0) and M <= 4096 or the jobs give 128
 * or more 32-column tiles (the workspace is then unused); else a partial launch over row chunks
 * and a fixed-order final launch through the workspace.  Deterministic either way. */
int nf4_lora_wgrad_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, int dtype,
                         void *workspace, size_t workspace_bytes, void *stream);
size_t nf4_lora_wgrad_multi_workspace(const nf4_lora_job *jobs, int njobs, int64_t m, int rank);

/* The gate | up pair of an MLP with the SwiGLU step fused into the GEMM epilogue, so the
 * [M, 2I] gate|up product never reaches memory.  gate_up: two weights of equal shape [I, K]
 * (gate, then up).  Forward: H[M, I] = silu(X Wg^T) * (X Wu^T), computed in fp32 from the fp32
 * accumulators and rounded once.  Backward (gate and up recomputed from X): with g, u those
 * products and sig = 1 / (1 + exp(-g)),
 *   dGU[:, 0:I]  = dH * u * sig * (1 + g (1 - sig)),   dGU[:, I:2I] = dH * g * sig,
 * the [M, 2I] gate|up gradient that nf4_linear_dx over the same pair consumes.  No workspace.
 * Replaces: the gate|up GEMM + gate_up_act_fwd_kernel / gate_up_act_bwd_kernel of
 *           FusedDecoderLayer (layer.py:266-296, 914-919, 1015-1019) and RecomputedMLP's
 *           gate, up, _swiglu_fwd / _swiglu_bwd (mlp.py:47-52, 65-70). */
int nf4_linear_swiglu_fwd(const void *x, int64_t m, int64_t ldx, const nf4_weight *gate_up,
                          void *h, int64_t ldh, int dtype, void *stream);
int nf4_linear_swiglu_bwd(const void *x, int64_t m, int64_t ldx, const nf4_weight *gate_up,
                          const void *dh, int64_t lddh, void *dgu, int64_t lddgu, int dtype,
                          void *stream);
/* Either of the two with the tiling pinned (NF4_TILE_*, never split; out = H or dGU, dh
 * ignored forward), for autotuning callers and tests of every tiling.
 * Replaces: the same reference code as the two above. */
int nf4_linear_swiglu_tiled(const void *x, int64_t m, int64_t ldx, const nf4_weight *gate_up,
                            void *out, int64_t ldo, const void *dh, int64_t lddh, int dtype,
                            void *stream, int backward, int tile);

/* ------------------------------- int8 input gradients of the MLP (off the fp16 parity path) */
/* The reference's T4 int8 backward (layer.py:299-442, 515-618, 992-1013): the input gradients
 * of down and of gate|up as int8 GEMMs with one scale per token and one per weight column.
 * Rounding to int8: ties away from zero, clamped to +-127 (layer.py:299-303).  Tolerance is the
 * reference's own (test_kernels.py:323-357): int8 operands within 0.6 scale of their value,
 * int8 products within 2e-2 of the largest fp32 result. */

/* scale[c] = max(largest |W[:, c]| over the stacked rows, 1e-20) / 127, W dequantized and
 * rounded to dtype (F16 / BF16): the fixed column scales of the transposed int8 weights.
 * Replaces: _col_scales (layer.py:598-615). */
size_t nf4_int8_colscale_workspace(const nf4_weight *ws, int nw);
int nf4_int8_colscale(const nf4_weight *ws, int nw, float *scale, int dtype, void *workspace,
                      size_t workspace_bytes, void *stream);

/* The stack as int8, transposed: q[c][r] = round(W[r][c] / scale[c]) with W the fp32 value
 * code[nib] * absmax; q row-major [cols, sum rows] with rows ldq bytes apart.  Rows and cols of
 * every weight multiples of 64.
 * Replaces: nf4_int8_t_kernel / _int8_t (layer.py:338-369, 579-595). */
int nf4_int8_weight_t(const nf4_weight *ws, int nw, const float *scale, int8_t *q, int64_t ldq,
                      void *stream);

/* The stack as int8 rows with one scale per row: s[r] = max(largest |W[r]|, 1e-20) / 127,
 * q[r][c] = round(W[r][c] * (127 / largest)).
 * Replaces: nf4_int8_rows_kernel / _int8_rows (layer.py:306-335, 565-576). */
int nf4_int8_weight_rows(const nf4_weight *ws, int nw, int8_t *q, int64_t ldq, float *s,
                         void *stream);

/* One int8 row per activation row (dtype F16 / BF16 / F32, cols a multiple of 8): s[r] =
 * max(largest |x[r]|, 1e-20) / 127, q[r][c] = round(x[r][c] * (127 / largest)).
 * Replaces: row_quant_kernel / _row_quant (layer.py:372-382, 555-562). */
int nf4_int8_rows(const void *x, int64_t rows, int64_t cols, int64_t ldx, int8_t *q, int64_t ldq,
                  float *s, int dtype, void *stream);

/* C[M, N] = A[M, K] . B[N, K]^T over int8 with exact int32 sums (K a multiple of 128, N of 4):
 * out_dtype NF4_I32 writes the sums, F16 / BF16 writes round(fp32(C) * sa[m] * sb[n]).
 * Workspace (int32 split-K partials): nf4_int8_gemm_workspace bytes.
 * Replaces: torch._int_mm and the scaling of its result (layer.py:1003, 1010-1012;
 *           test_kernels.py:348, 353). */
size_t nf4_int8_gemm_workspace(int64_t m, int64_t n, int64_t k);
int nf4_int8_gemm(const int8_t *a, int64_t m, int64_t lda, const int8_t *b, int64_t n,
                  int64_t ldb, int64_t k, const float *sa, const float *sb, void *c, int64_t ldc,
                  int out_dtype, void *workspace, size_t workspace_bytes, void *stream);

/* SwiGLU backward on the int32 sums acc[M, I] of dh8 . Wd8^T with per-row int8 requantization:
 * dh = fp32(acc) * sd[m] * cs[j]; with g, u the saved gate | up ([M, 2I], dtype) and
 * sig = 1 / (1 + exp(-g)): q[m][j] = round(dh u sig (1 + g (1 - sig)) * 127 / peak),
 * q[m][I + j] = round(dh g sig * 127 / peak), sq[m] = peak / 127, peak the row's largest
 * |gradient| (at least 1e-20).
 * Replaces: gate_up_act_bwd_i8_kernel (layer.py:414-442). */
int nf4_int8_swiglu_bwd(const int32_t *acc, int64_t m, int64_t inter, int64_t ldacc,
                        const float *sd, const float *cs, const void *gu, int64_t ldgu, int8_t *q,
                        int64_t ldq, float *sq, int dtype, void *stream);

/* ------------------------------------------- the projection's neighbours: RMSNorm, RoPE */

/* One row per token (contiguous [rows, cols] tensors, cols a multiple of 8, at most 8192):
 * h = x (+ d), rstd[r] = 1 / sqrt(mean(h^2) + eps), y = w * (h * rstd) in fp32 rounded once to
 * dtype; w is fp32 [cols].  x is the residual stream in res_dtype (NF4_F32, or dtype); d (the
 * o_proj output, may be NULL), y, oq and ov are in dtype.
 * LoRA dropout (drop_mode 1 or 2) also writes the dropout inputs oq = y * keep_q * scale_q and
 * ov = y * keep_v * scale_v (scale = 1 / (1 - p)), each rounded once.  The keep masks live
 * packed: packed[r][0][j] bit k = keep_q of element 8 j + k, packed[r][1][j] the same for v
 * ([rows][2][cols / 8] bytes).  Mode 1 reads one-byte 0/1 masks keep_q, keep_v [keep_rows,
 * cols] (8-byte aligned) at row src_rows[r] (row r when src_rows is NULL, which needs
 * keep_rows >= rows: the token's row of masks drawn over a padded batch) and writes their bits
 * to packed; a src_rows entry outside [0, keep_rows) reads as all dropped.  Mode 2 reads
 * packed.
 * Replaces: add_rmsnorm_fwd_kernel with _pack_bits / _unpack_bits
 *           (/root/reference/solution/layer.py:76-132). */
int nf4_add_rmsnorm(const void *x, int res_dtype, const void *d, const float *w, void *y,
                    float *rstd, const uint8_t *keep_q, const uint8_t *keep_v,
                    const int64_t *src_rows, int64_t keep_rows, uint8_t *packed, int drop_mode, float scale_q,
                    float scale_v, void *oq, void *ov, int64_t rows, int64_t cols, float eps,
                    int dtype, void *stream);

/* The gradient of the above: g = dy (+ dq * keep_q * scale_q + dv * keep_v * scale_v, the
 * keep bits read from packed), h = x (+ d) recomputed, h^ = h * rstd,
 * dx = rstd * (g w - h^ * mean(g w h^)) (+ dres).  dy, dq, dv and d in dtype; x, dres and dx in
 * res_dtype.  dy, dq/dv (together, with packed), d and dres may be NULL.
 * Replaces: rmsnorm_bwd_lora_kernel (/root/reference/solution/layer.py:135-164). */
int nf4_rmsnorm_bwd(const void *dy, const void *dq, const void *dv, const uint8_t *packed,
                    float scale_q, float scale_v, const void *x, int res_dtype, const void *d,
                    const float *w, const float *rstd, const void *dres, void *dx, int64_t rows,
                    int64_t cols, int dtype, void *stream);

/* Rotary embedding of the finished q|k|v projection (qkv [tokens, ld_qkv], columns n_heads q
 * heads, n_kv k heads, n_kv v heads of head_dim each; the LoRA terms are already in it, added by
 * nf4_linear_fwd's epilogue): per pair i < head_dim/2, lo' = lo cos[i] - hi sin[i],
 * hi' = hi cos[half + i] + lo sin[half + i] on q and k in fp32 (cos, sin fp32 [tokens, head_dim]),
 * q, k, v written as [tokens, n_heads, head_dim] (k, v expanded to every query head of their
 * group), and the unexpanded k, v to k_cache / v_cache [tokens, n_kv, head_dim] when given.
 * Replaces: qkv_lora_rope_kernel (/root/reference/solution/layer.py:167-218) minus its LoRA
 *           add (layer.py:190-193, 208-211), which moved into the GEMM. */
int nf4_qkv_rope(const void *qkv, int64_t ld_qkv, const float *cos_t, const float *sin_t,
                 void *q, void *k, void *v, void *k_cache, void *v_cache, int64_t tokens,
                 int n_heads, int n_kv, int head_dim, int dtype, void *stream);

/* The gradient of the above into dqkv [tokens, ld_dqkv] (q|k|v columns): the transposed
 * rotation of dq and of dk summed over each group's expanded heads; dv summed the same way.
 * Replaces: qkv_rope_bwd_kernel (/root/reference/solution/layer.py:221-263). */
int nf4_qkv_rope_bwd(const void *dq, const void *dk, const void *dv, const float *cos_t,
                     const float *sin_t, void *dqkv, int64_t ld_dqkv, int64_t tokens, int n_heads,
                     int n_kv, int head_dim, int dtype, void *stream);

/* -------------------------------------------------------------------------- small helpers */

/* out[rows, cols] = silu(gate) * up, and its gradient (the SwiGLU step between the gate/up and
 * down GEMMs of RecomputedMLP, mlp.py:26-39, 52, 70; example kernels swiglu.py:15-37).
 * gate/up (and dgate/dup) rows are ld_gu elements apart, so they can be the two halves of the
 * stacked gate|up GEMM output; out / grad rows are ld_h apart. */
int nf4_swiglu_fwd(const void *gate, const void *up, int64_t ld_gu, void *out, int64_t ld_h,
                   int64_t rows, int64_t cols, int dtype, void *stream);
int nf4_swiglu_bwd(const void *grad, int64_t ld_h, const void *gate, const void *up,
                   int64_t ld_gu, void *dgate, void *dup, int64_t rows, int64_t cols, int dtype,
                   void *stream);

/* out[N] = sum over rows of dY[M, N] (fp32): the bias gradient of NF4Linear.backward
 * (nf4.py:100-101). */
int nf4_bias_grad(const void *dy, int64_t m, int64_t n, int64_t lddy, float *out, int dtype,
                  void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NF4_MI355X_H */
