/* aq: MI355X (gfx950) weight-quantized matmul kernels behind a plain C ABI.
 *
 * Every entry point takes caller-owned device pointers, shape scalars and a hipStream_t (passed as void*, so this
 * header needs no HIP include), enqueues its kernels on that stream without synchronising, allocates nothing and
 * returns an aq_status. Layouts are the reference's packed layouts:
 *   Q4W  wq uint32 [N, K/8]: element k of row n in bits 4*(k%8) of word k/8, 4-bit two's complement
 *        (value ((nib ^ 8) - 8) * ws[n, k/G]); ws fp16 [N, K/G].
 *   T2W  w uint32 [K/16, N] (transposed): code of (n, k) in bits 2*(k%16) of word (k/16)*N + n, value
 *        (code - 1) * s[k/128, n]; s fp16 [K/128, N].
 *   X2H  uint32 [K/2]: fp16 pairs, the even k in the low half.
 * fp16 values are passed as uint16_t bit patterns. Reference citations are file:line in adityaGoCT/mojo-adreno.
 */
#ifndef AQ_H
#define AQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  AQ_OK = 0,
  AQ_ERR_SHAPE = 1,    /* a size is zero/negative, or not a multiple the layout requires */
  AQ_ERR_GROUP = 2,    /* group size not a multiple of 8, or K not a multiple of it */
  AQ_ERR_ALIGN = 3,    /* a pointer is not 16-byte aligned */
  AQ_ERR_LAUNCH = 4,   /* the HIP launch failed (hipGetLastError) */
  AQ_ERR_NULL = 5,     /* a required pointer is NULL */
  AQ_ERR_CAPACITY = 6, /* a size exceeds what the kernel's on-chip staging holds */
  AQ_ERR_ARG = 7       /* any other invalid argument */
} aq_status;

/* Human-readable text of a status code (static storage). */
const char* aq_status_string(int status);

/* Library version, as major*10000 + minor*100 + patch. */
int aq_version(void);

/* ---- int4 (Q4W) matrix-vector products, decode ------------------------------------------------------------------
 * y[t, n] = (add ? y[t, n] : 0) + sum_k W[n, k] * x[t, k] for t < tokens, fp32 x [tokens, K] and y [tokens, N].
 * tokens = 1 is the decode GEMV; tokens <= 8 the few-token form. Every weight word is read once per launch for
 * all tokens.
 * Replaces: gemv_q4 (llama/kernels/gemv_q4.mojo:13-30, G=64), gemv_add_q4 (llama/kernels/gemv_add_q4.mojo:13-30,
 * add=1), lk.gemv_q4[B] (lfm2/kernels/lk.mojo:134-143, G=32), moek.p_gemv_q4 / t_gemv_q4
 * (qwen3moe/kernels/moek.mojo:273-281,528-545: tokens, add).
 * Requires K % 32 == 0, K % group == 0, group % 8 == 0, tokens in 1..8, K*tokens <= 32768, 16-byte aligned wq/x. */
int aq_gemv_q4(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int64_t n, int64_t k,
               int32_t group, int32_t tokens, int32_t add, void* stream);

/* a[t, j] = silu(W[j] . x[t]) * (W[f + j] . x[t]) for j < f over the fused gate|up matrix W [2f, K].
 * Replaces: lk.gate_up_q4[B] (lfm2/kernels/lk.mojo:154-167). Same requirements as aq_gemv_q4. */
int aq_gate_up_q4(const uint32_t* wq, const uint16_t* ws, const float* x, float* a, int64_t f, int64_t k,
                  int32_t group, int32_t tokens, void* stream);

/* ---- int4 (Q4W) GEMM on MFMA, prefill ------------------------------------------------------------------------------
 * Y[m, n] = (add ? Y[m, n] : 0) + sum_k X[m, k] * W[n, k] with X [M, K] fp16 (x_is_f32 = 0) or fp32 (x_is_f32 = 1,
 * rounded to fp16 on staging), Y fp32 [M, N]; W dequantised to fp16, fp32 accumulation (rel 1e-2 bar).
 * Replaces: p_gemm_q4 (llama/kernels/prefill/p_gemm_q4.mojo:106-142, G=64, fp32 X) and lk.gemm_q4
 * (lfm2/kernels/lk.mojo:458-495, G=32). The reference needs M, N % 128 and K % 16; here any M, N >= 1 and
 * K % 32 == 0, K % group == 0, group % 8 == 0, 16-byte aligned x/wq/y, each operand < 2 GiB.
 * workspace: caller-owned device memory for split-K partials, aq_gemm_q4_workspace_bytes(m, n, k) bytes (16-byte
 * aligned); NULL or smaller runs one pass over K (correct, fewer workgroups). Calls sharing a workspace must be
 * ordered on one stream. */
int aq_gemm_q4(const void* x, int32_t x_is_f32, const uint32_t* wq, const uint16_t* ws, float* y, int64_t m,
               int64_t n, int64_t k, int32_t group, int32_t add, void* workspace, int64_t workspace_bytes,
               void* stream);

/* Workspace bytes aq_gemm_q4 uses for this shape (0 when it runs without split-K). No counterpart in the reference
 * (its kernels need no scratch). */
int64_t aq_gemm_q4_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* ---- ternary (T2W) GEMM on MFMA, prefill ----------------------------------------------------------------------------
 * Y[m, n] = (add ? Y : 0) + sum_k X[m, k] * (code(k, n) - 1) * s[k/128, n], X fp16 or fp32 (rounded to fp16),
 * T2W w [K/16, N], s fp16 [K/128, N], fp32 accumulation (rel 1e-2 bar). Requires K % 128 == 0.
 * Replaces: p_gemm_t2 / p_gemm_t2v (bonsai/kernels/prefill.mojo:155-171,174-313; M, N % 128 there), and the
 * per-shape tile table gemm_table.gemm_t2 (qwen3/gemm_table.mojo:9-57): one kernel plans its own tiles and split.
 * workspace as for aq_gemm_q4, aq_gemm_t2_workspace_bytes(m, n, k) bytes. */
int aq_gemm_t2(const void* x, int32_t x_is_f32, const uint32_t* w, const uint16_t* s, float* y, int64_t m, int64_t n,
               int64_t k, int32_t add, void* workspace, int64_t workspace_bytes, void* stream);
int64_t aq_gemm_t2_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* ---- ternary (T2W) matrix-vector products, decode ---------------------------------------------------------------
 * y[n] = sum_k (code(k, n) - 1) * s[k/128, n] * x[k], x as X2H fp16 pairs [K/2], T2W w [K/16, N], s fp16 [K/128, N],
 * fp32 accumulation (the reference accumulates groups in fp16). Requires K % 128 == 0, 16-byte aligned w.
 * Replaces: packed_linear + packed_reduce (bonsai/kernels/kernels.mojo:283-325,437-448) in one launch.
 * workspace: aq_t2_gemv_workspace_bytes(n, k) bytes, zero-filled before its first use: its first 64 KiB hold
 * per-column-tile arrival counters (every call leaves them at zero again), the rest split-K partials. Keep it for
 * aq_t2_gemv only; calls sharing it must be ordered on one stream. NULL runs without splitting K. */
int aq_t2_gemv(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* y, int64_t n, int64_t k,
               void* workspace, int64_t workspace_bytes, void* stream);
int64_t aq_t2_gemv_workspace_bytes(int64_t n, int64_t k);

/* partials[g, n] = sum over k in [1024 g, 1024 g + 1024) of the products above, g < ceil(K/1024).
 * Replaces: packed_linear (bonsai/kernels/kernels.mojo:283-325; its grid (ceil(N/64), ceil(K/1024))). */
int aq_t2_packed_linear(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* partials, int64_t n,
                        int64_t k, void* stream);

/* y[n] = sum_{g < groups} partials[g, n], in g order. Replaces: packed_reduce (bonsai/kernels/kernels.mojo:437-448). */
int aq_t2_packed_reduce(const float* partials, float* y, int64_t n, int32_t groups, void* stream);

/* ---- X2H producers (fp32 -> fp16 pairs, round to nearest even; even k in the low half) ------------------------ */
/* q[i] = pack(x[2i], x[2i+1]), count = number of floats. Replaces: pack_half (qwen3/kernels/qwen3k.mojo:45-48). */
int aq_pack_half(const float* x, uint32_t* q, int64_t count, void* stream);
/* q[row] = pack(x[row] * rsqrt(mean(x[row]^2) + eps) * w), rows of n. Replaces: rmsnorm_pack
 * (qwen3/kernels/qwen3k.mojo:30-42, eps 1e-6, one row). */
int aq_rmsnorm_pack(const float* x, const float* w, uint32_t* q, int64_t rows, int64_t n, float eps, void* stream);
/* q[row] = pack(silu(gate) * up), gu rows = gate (n) | up (n). Replaces: swiglu_pack (qwen3/kernels/qwen3k.mojo:51-59). */
int aq_swiglu_pack(const float* gu, uint32_t* q, int64_t rows, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AQ_H */
