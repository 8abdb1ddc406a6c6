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
 * tokens = 1 is the decode GEMV; tokens <= 16 the few-row form (a weight row read once for all rows). Every weight
 * word is read once per launch for all tokens.
 * Replaces: gemv_q4 (llama/kernels/gemv_q4.mojo:13-30, G=64), gemv_add_q4 (llama/kernels/gemv_add_q4.mojo:13-30,
 * add=1), lk.gemv_q4[B] (lfm2/kernels/lk.mojo:134-143, G=32), moek.p_gemv_q4 / t_gemv_q4
 * (qwen3moe/kernels/moek.mojo:273-281,528-545: tokens, add), and the few-row products rows_q4 (lfm2/kernels/dsk.mojo:
 * 97-119, count <= 12, speculative verify).
 * Requires K % 32 == 0, K % group == 0, group % 8 == 0, tokens in 1..16, K * (tokens rounded up to 1, 2, 4, 8 or 16)
 * <= 32768, 16-byte aligned wq/x. */
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

/* aq_gemm_q4 without a workspace argument and without any allocation: the split-K partials live in a static device
 * array of AQ_GEMM_NOALLOC_SCRATCH_BYTES, one per GPU, held until the process ends. Same plan, kernels and result as
 * aq_gemm_q4 given a large enough workspace (bit for bit). A shape whose partials exceed the array (at most
 * aq_gemm_q4_workspace_bytes(m, n, k) bytes) is refused with AQ_ERR_CAPACITY; `stream` must belong to the current
 * device (else AQ_ERR_ARG). Every call on one GPU shares its array, so calls that overlap on one GPU race: order them
 * on one stream. No counterpart in the reference; it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). */
#define AQ_GEMM_NOALLOC_SCRATCH_BYTES (32ll << 20)
int aq_gemm_q4_noalloc(const void* x, int32_t x_is_f32, const uint32_t* wq, const uint16_t* ws, float* y, int64_t m,
                       int64_t n, int64_t k, int32_t group, int32_t add, void* stream);

/* ---- ternary (T2W) GEMM on MFMA, prefill ----------------------------------------------------------------------------
 * Y[m, n] = (add ? Y : 0) + sum_k X[m, k] * (code(k, n) - 1) * s[k/128, n], X fp16 or fp32 (rounded to fp16),
 * T2W w [K/16, N], s fp16 [K/128, N], fp32 accumulation (rel 1e-2 bar). Requires K % 128 == 0.
 * Replaces: p_gemm_t2 / p_gemm_t2v (bonsai/kernels/prefill.mojo:155-171,174-313; M, N % 128 there), and the
 * per-shape tile table gemm_table.gemm_t2 (qwen3/gemm_table.mojo:9-57): one kernel plans its own tiles and split.
 * workspace as for aq_gemm_q4, aq_gemm_t2_workspace_bytes(m, n, k) bytes. */
int aq_gemm_t2(const void* x, int32_t x_is_f32, const uint32_t* w, const uint16_t* s, float* y, int64_t m, int64_t n,
               int64_t k, int32_t add, void* workspace, int64_t workspace_bytes, void* stream);
int64_t aq_gemm_t2_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* ---- mixture of experts ----------------------------------------------------------------------------------------------
 * Grouped int4 GEMM over experts. Work tile it < ntiles[0] (device) is (tiles[2it] = expert e, tiles[2it+1] = first
 * grouped row g0); its tm rows g0 .. g0+tm-1 read X row src[g] (a token of x [x_rows, K]; -1 = padding row, zeros)
 * or row g itself when src is NULL. W holds the experts stacked: expert e's n rows start at row e*n (Q4W
 * [experts*n, K/8], fp16 scales [experts*n, K/group]).
 *   swiglu = 0: out fp32 [rows_total, n], out[g] = X_g . W_e^T.
 *   swiglu = 1: W_e rows are gate (n/2) | up (n/2); out fp16 [rows_total, n/2], out[g, j] = silu(g_j) * u_j.
 * max_tiles bounds the grid (aq_moe_group_max_tiles); tm a multiple of 16 up to 112. x fp16 (x_is_f32 = 0) or fp32.
 * Replaces: p_gemm_q4g (lfm2moe/kernels/mk.mojo:208-257) with p_gather (:164-176) and p_silu_mul (:179-186) folded in,
 * and t_moe_gate_up / t_moe_down (qwen3moe/kernels/moek.mojo:560-608). */
int aq_moe_gemm_q4(const void* x, int32_t x_is_f32, int64_t x_rows, const int32_t* src, const uint32_t* wq,
                   const uint16_t* ws, int64_t experts, int64_t n, int64_t k, int32_t group, const int32_t* tiles,
                   const int32_t* ntiles, int32_t max_tiles, int32_t tm, int64_t rows_total, int32_t swiglu, void* out,
                   void* stream);

/* Top-k routing: per token, the k largest of `experts` logits (descending; the lowest index among equals) and their
 * weights exp(l_k - l_max) / sum_top exp(l_j - l_max) (softmax, top-k, renormalise). experts <= 256, topk <= 8.
 * Replaces: route / p_route (qwen3moe/kernels/moek.mojo:156-197,385-425). */
int aq_moe_route(const float* logits, int32_t* ids, float* weights, int64_t tokens, int32_t experts, int32_t topk,
                 void* stream);

/* aq_moe_route, and with it x [tokens, d] fp32 rounded to fp16 pairs xq [tokens, d/2] (the grouped GEMM's input) in
 * the same launch: one wave per token does both. d % 8 == 0, x and xq 16-byte aligned. Replaces: route / p_route
 * (as aq_moe_route) followed by the fp32 -> fp16 rounding of the MoE block's input (lfm2moe/kernels/mk.mojo:164-176
 * gathers fp32 rows; this build's grouped GEMM reads fp16). */
int aq_moe_route_pack(const float* logits, int32_t* ids, float* weights, int64_t tokens, int32_t experts,
                      int32_t topk, const float* x, uint32_t* xq, int64_t d, void* stream);

/* Grouping of the routed entries i = t*topk + k by expert (one workgroup, deterministic): counts[e]; offs[e] =
 * exclusive prefix sum of the counts padded to multiples of tm (offs[experts] = rows used); slot[i] = grouped row
 * (ascending i within an expert); src[row] = token (-1 on padding and unused rows < max_rows); work tiles (e, row)
 * every tm rows of each expert, in expert order, and their number ntiles[0]. max_rows >= aq_moe_group_max_rows,
 * max_tiles >= aq_moe_group_max_tiles. A token may name one expert more than once: every entry is counted and
 * entries of one expert keep ascending i (a slower ordered scan then runs in the same launch); an id outside
 * [0, experts) gets slot -1. Replaces: p_group (lfm2moe/kernels/mk.mojo:123-161). */
int aq_moe_group(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts, int32_t tm, int32_t* counts,
                 int32_t* offs, int32_t* slot, int32_t* src, int64_t max_rows, int32_t* tiles, int32_t max_tiles,
                 int32_t* ntiles, void* stream);
int64_t aq_moe_group_max_rows(int64_t tokens, int32_t topk, int32_t experts, int32_t tm);
int32_t aq_moe_group_max_tiles(int64_t tokens, int32_t topk, int32_t experts, int32_t tm);

/* Per-expert lists of entries: lists[e*cap + r] = the r-th entry i (ascending, repeated ids included) with
 * ids[i] == e, counts[e]; with items != NULL also the work items (e, c) for c = 0, items_tt, ... < counts[e] in expert
 * order and nitems[0].
 * scratch: >= (experts + 1) + 4 * tokens * topk + 1 ints of device memory. Replaces: p_expert_lists and
 * p_expert_items (qwen3moe/kernels/moek.mojo:432-442,548-557; cap = PMAX there). */
int aq_moe_expert_lists(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts, int32_t cap,
                        int32_t* lists, int32_t* counts, int32_t items_tt, int32_t* items, int32_t max_items,
                        int32_t* nitems, int32_t* scratch, int64_t scratch_ints, void* stream);

/* y[t, c] = (add ? y[t, c] : 0) + sum_{k < topk} weights[t, k] * yd[slot[t*topk + k], c], k in order; slot NULL means
 * row t*topk + k. Replaces: p_combine (lfm2moe/kernels/mk.mojo:189-199) and, with slot NULL and add = 1, p_moe_sum
 * (qwen3moe/kernels/moek.mojo:479-488). d % 4 == 0; a slot outside [0, yd_rows) contributes nothing. */
int aq_moe_combine(const float* yd, int64_t yd_rows, const int32_t* slot, const float* weights, float* y,
                   int64_t tokens, int64_t d, int32_t topk, int32_t add, void* stream);

/* Decode (one token): a[e, j] = silu(W[ids[e]*2f + j] . x) * (W[ids[e]*2f + f + j] . x), e < topk, j < f.
 * An id outside [0, experts) gives a[e] = 0 (the reference does not check).
 * Replaces: moe_gate_up (qwen3moe/kernels/moek.mojo:200-210; lfm2moe/kernels/mk.mojo:94-104). */
int aq_moe_gate_up_q4(const uint32_t* wq, const uint16_t* ws, int64_t experts, const int32_t* ids, const float* x,
                      float* a, int64_t f, int64_t k, int32_t group, int32_t topk, void* stream);

/* Decode: y[r] = (add ? y[r] : 0) + sum_e weights[e] * W[ids[e]*d + r] . a[e], e in order.
 * An id outside [0, experts) contributes nothing.
 * Replaces: moe_down (qwen3moe/kernels/moek.mojo:213-223, add = 1; lfm2moe/kernels/mk.mojo:107-118, add = 0). */
int aq_moe_down_q4(const uint32_t* wq, const uint16_t* ws, int64_t experts, const int32_t* ids, const float* weights,
                   const float* a, float* y, int64_t d, int64_t f, int32_t group, int32_t topk, int32_t add,
                   void* stream);

/* Router: y[t, r] = W[r] . x[t], fp32 W [n, k]. Replaces: gemv_f32 / p_gemv_f32 (qwen3moe/kernels/moek.mojo:143-153,
 * 284-295). */
int aq_gemv_f32(const float* w, const float* x, float* y, int64_t n, int64_t k, int32_t tokens, void* stream);

/* ---- ternary (T2W) matrix-vector products, decode ---------------------------------------------------------------
 * y[n] = sum_k (code(k, n) - 1) * s[k/128, n] * x[k], x as X2H fp16 pairs [K/2], T2W w [K/16, N], s fp16 [K/128, N],
 * fp32 accumulation (the reference accumulates groups in fp16). Requires K % 128 == 0, 16-byte aligned w.
 * Replaces: packed_linear + packed_reduce (bonsai/kernels/kernels.mojo:283-325,437-448) in one launch: each workgroup
 * owns a block of columns over all of K and reduces inside itself, so no cross-workgroup step is needed. K <= 32768.
 * workspace is unused (aq_t2_gemv_workspace_bytes returns 0); it is kept in the signature for callers that pass one. */
int aq_t2_gemv(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* y, int64_t n, int64_t k,
               void* workspace, int64_t workspace_bytes, void* stream);
int64_t aq_t2_gemv_workspace_bytes(int64_t n, int64_t k);

/* Ternary output head with greedy argmax on the device, one launch: logits = the aq_t2_gemv product over the
 * vocabulary rows, then *token = the first index of the largest logit, or -1 when any logit is NaN or infinite,
 * hist[*pos] = *token when 0 <= *pos < hist_cap (hist may be NULL), *pos += advance. cand: aq_t2_head_candidates(n, k)
 * 8-byte slots (8-byte aligned): an argmax key per workgroup, then the arrival counters in the last
 * AQ_HEAD_ARRIVAL_SLOTS slots, as in aq_head_argmax_q4 (zero before the first call, left zero; calls sharing a cand
 * ordered on one stream). Replaces: packed_head with
 * select = 1 (bonsai/kernels/kernels.mojo:451-517: logits plus per-64-lane (best, index, nonfinite) candidates) and
 * the host's greedy() over them (bonsai/bonsai_vk.c:506-515: largest value, lowest index on ties; a nonfinite flag
 * stops it with "nonfinite logits"). */
int aq_t2_head_argmax(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* logits, int64_t n, int64_t k,
                      uint64_t* cand, int64_t cand_cap, int32_t* token, int32_t* pos, int32_t* hist, int32_t hist_cap,
                      int32_t advance, void* stream);
int64_t aq_t2_head_candidates(int64_t n, int64_t k);

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

/* ---- Llama decode step (one token): the kernels around the int4 GEMVs -------------------------------------------
 * The reference's step (llama/model.mojo:128-166) launches embed, then per layer rmsnorm, gemv_q4 (qkv), rope_kv,
 * attention, gemv_add_q4 (o), rmsnorm, gemv_q4 (gate|up), silu_mul, gemv_add_q4 (down), then rmsnorm and the lm_head;
 * the host then scans the logits for the argmax (llama/llama.mojo:72-75). Here the norms and silu_mul are fused into
 * the GEMVs that consume them, RoPE and the cache append into attention, and the argmax runs on the device, so a step
 * is 1 + 5 per layer + 2 launches. Token and position live in device memory (int32), so a captured step replays
 * without host work. */

/* y = W . rmsnorm(x), rmsnorm(x) = x * (1 / sqrt(mean(x^2) + eps)) * norm_w (fp16 [K]), per token; as aq_gemv_q4
 * otherwise (add = 0). Replaces: rmsnorm (llama/kernels/rmsnorm.mojo:17-35) + gemv_q4 (gemv_q4.mojo:13-30), the pair
 * at llama/model.mojo:146-147. norm_w 16-byte aligned. */
int aq_rmsnorm_gemv_q4(const uint32_t* wq, const uint16_t* ws, const float* x, const uint16_t* norm_w, float eps,
                       float* y, int64_t n, int64_t k, int32_t group, int32_t tokens, void* stream);

/* a = silu(W_gate . rmsnorm(x)) * (W_up . rmsnorm(x)), W = gate|up [2f, K]. Replaces: rmsnorm + gemv_q4 (wgu) +
 * silu_mul (llama/kernels/silu_mul.mojo:9-12), llama/model.mojo:151-153. */
int aq_rmsnorm_gate_up_q4(const uint32_t* wq, const uint16_t* ws, const float* x, const uint16_t* norm_w, float eps,
                          float* a, int64_t f, int64_t k, int32_t group, int32_t tokens, void* stream);

/* x[i] = table[*token, i] as fp32, table fp16 [vocab, d], d % 8 == 0 (a token outside [0, vocab) reads row 0).
 * Replaces: embed (llama/kernels/embed.mojo:9-11; llama/model.mojo:142-143, which picks one of 4 table chunks). */
int aq_embed_f16(const uint16_t* table, int64_t vocab, int64_t d, const int32_t* token, float* x, void* stream);

/* Attention of the token at position p = *pos: RoPE (rotate_half, cos/sin fp32 [max_pos, head_dim/2]) on q and k of
 * qkv fp32 [(heads + 2 kv_heads) * head_dim]; k and v stored at row p of k_cache/v_cache fp16 [kv_heads, max_pos,
 * head_dim]; out[h] = softmax_s(q_h . k_s / sqrt(head_dim)) . v_s over s <= p, fp32 [heads * head_dim]. head_dim = 64,
 * heads / kv_heads in {1, 2, 4, 8}, LDS (heads / kv_heads) * (max_pos + 2120) floats <= 160 KB (max_pos <= 8120 for
 * 4 query heads per KV head). A p outside [0, max_pos) writes zeros
 * and leaves the cache alone. Replaces: rope_kv (llama/kernels/rope_kv.mojo:18-45) + attention (attention.mojo:19-66),
 * llama/model.mojo:148-150; the reference caches fp32. */
int aq_attn_decode(const float* qkv, const float* cos_tab, const float* sin_tab, uint16_t* k_cache, uint16_t* v_cache,
                   const int32_t* pos, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_pos, float* out,
                   void* stream);

/* Split attention (flash decoding), the decode step's form of aq_attn_decode: the positions of each KV head are cut
 * into `splits` spans of ceil(max_pos / splits) rounded up to 64, one workgroup each (kv_heads * splits workgroups
 * instead of kv_heads), and each writes the partial softmax state of its span for every query head h:
 *   parts: o [heads][splits][64] (sum over the span of e^(s - m) v), then (m, l) [heads][splits][2] (the span's max
 *   score and sum of e^(s - m)); a span past the position holds m = -inf, l = 0, o = 0.
 * RoPE and the cache append are as in aq_attn_decode. aq_attn_out_q4 combines the spans. 1 <= splits <=
 * AQ_ATTN_MAX_SPLITS; (heads / kv_heads) * span floats of LDS <= 64 KB. No counterpart in the reference (its attention
 * is one workgroup per head, llama/kernels/attention.mojo:19-66); same result to fp32 rounding. */
#define AQ_ATTN_MAX_SPLITS 8
int aq_attn_decode_split(const float* qkv, const float* cos_tab, const float* sin_tab, uint16_t* k_cache,
                         uint16_t* v_cache, const int32_t* pos, int32_t heads, int32_t kv_heads, int32_t head_dim,
                         int32_t max_pos, int32_t splits, float* parts, void* stream);

/* y += W . att, where att [k = heads * 64] is combined from the split-attention states while x is staged:
 * att[h, d] = sum_c e^(m_c - M) o_c[d] / sum_c e^(m_c - M) l_c, M = max_c m_c. Otherwise aq_gemv_q4 (add = 1,
 * tokens = 1). Replaces: gemv_add_q4 of the attention output (llama/model.mojo:150, llama/kernels/gemv_add_q4.mojo:
 * 13-30), with the split combine folded in. */
int aq_attn_out_q4(const uint32_t* wq, const uint16_t* ws, const float* parts, int32_t splits, float* y, int64_t n,
                   int64_t k, int32_t group, void* stream);

/* Final norm, lm_head and greedy argmax: logits = W . rmsnorm(x) (norm_w NULL: x as given), then *token = the first
 * index of the largest logit, hist[*pos] = *token when 0 <= *pos < hist_cap (hist may be NULL), *pos += advance.
 * One launch: every workgroup (at most 1024) leaves its best argmax key in cand and counts itself on arrival
 * counters kept in cand's last AQ_HEAD_ARRIVAL_SLOTS slots; the workgroup that arrives last writes the token and sets
 * the counters back to zero.
 * cand: device scratch of cand_cap 8-byte slots (8-byte aligned; AQ_HEAD_CANDIDATES is enough for any vocab), whose
 * last AQ_HEAD_ARRIVAL_SLOTS slots must be zero before the first call (a zero-filled buffer) and are left zero by
 * every call; calls sharing a cand must be ordered on one stream. NaN logits never win, as in the reference's `logits[i] > logits[best]` scan
 * (which differs only when logit 0 itself is NaN: it then returns 0).
 * Replaces: Llama.head (llama/model.mojo:160-166) and the host argmax scan (llama/llama.mojo:72-75). */
#define AQ_HEAD_CANDIDATES 4096
#define AQ_HEAD_ARRIVAL_SLOTS 17
int aq_head_argmax_q4(const uint32_t* wq, const uint16_t* ws, const float* x, const uint16_t* norm_w, float eps,
                      float* logits, int64_t vocab, int64_t k, int32_t group, uint64_t* cand, int64_t cand_cap,
                      int32_t* token, int32_t* pos, int32_t* hist, int32_t hist_cap, int32_t advance, void* stream);

/* ---- Q6_K tied head / embedding (Q6W: q [rows, cols/256, 208] bytes, 16-byte aligned, d fp16 [rows, cols/256], as
 * aq_gguf_q6_k_to_q6w writes them; cols % 256 == 0, rows * cols / 256 * 208 < 2^31) ---- */

/* y[r] = E[r] . x, E the dequantized Q6W matrix ((d * sc) * (q - 32)), x fp32 [cols] (16-byte aligned), y fp32 [rows].
 * Replaces: head_q6 (lfm2/kernels/lk.mojo:179-191, q6_chunk :88-129). */
int aq_gemv_q6(const uint8_t* q, const uint16_t* d, const float* x, float* y, int64_t rows, int64_t cols,
               void* stream);

/* Final norm, Q6_K head and greedy argmax, one launch: logits = E . rmsnorm(x) (norm_w NULL: x as given), then as
 * aq_head_argmax_q4: *token = the first index of the largest logit (NaN never wins), hist[*pos] = *token when
 * 0 <= *pos < hist_cap, *pos += advance. cand: aq_head_q6_candidates(rows, cols) <= AQ_HEAD_CANDIDATES 8-byte slots
 * (8-byte aligned): an argmax key per workgroup, then the arrival counters in the last AQ_HEAD_ARRIVAL_SLOTS slots,
 * as in aq_head_argmax_q4 (zero before the first call, left zero; calls sharing a cand ordered on one stream). Replaces: head_q6 + argmax (lfm2/kernels/lk.mojo:179-221: lowest index among equal maxima). */
int aq_head_argmax_q6(const uint8_t* q, const uint16_t* d, const float* x, const uint16_t* norm_w, float eps,
                      float* logits, int64_t rows, int64_t cols, uint64_t* cand, int64_t cand_cap, int32_t* token,
                      int32_t* pos, int32_t* hist, int32_t hist_cap, int32_t advance, void* stream);
int64_t aq_head_q6_candidates(int64_t rows, int64_t cols);

/* x[t] = the dequantized row ids[t] of the Q6W matrix, fp32 [ntok, cols] (16-byte aligned), bit-exact
 * (d * sc) * (q - 32); ids outside [0, rows) read row 0. ids: device int32 [ntok], ntok <= 65535.
 * Replaces: embed_q6 (lfm2/kernels/lk.mojo:224-232). */
int aq_embed_q6(const uint8_t* q, const uint16_t* d, int64_t rows, int64_t cols, const int32_t* ids, int32_t ntok,
                float* x, void* stream);

/* ---- measurement ---------------------------------------------------------------------------------------------------
 * Streaming read: every 16 bytes of p [bytes] read once with the matrix-vector kernels' streaming cache policy,
 * nothing else computed, by `blocks` workgroups of 4 waves (0: one 8 KB page each, at most
 * AQ_STREAM_READ_MAX_BLOCKS); wave w of workgroup b writes the XOR of the 32-bit words it read to sink[4 b + w], so
 * the XOR of sink[0 .. 4 blocks) is the XOR of the whole buffer. bytes % 16 == 0, bytes < 2^31,
 * blocks <= AQ_STREAM_READ_MAX_BLOCKS. No counterpart in the reference: a launch over a weight matrix's bytes is the
 * ceiling its matrix-vector product is measured against. */
#define AQ_STREAM_READ_MAX_BLOCKS 8192
int aq_stream_read(const void* p, int64_t bytes, int32_t blocks, uint32_t* sink, void* stream);

/* ---- weight-format converters (host code: host pointers, synchronous, no GPU) ----------------------------------
 * They write the layouts above from the reference's source formats, byte for byte as the reference's converters do. */

/* Q4W from fp16 weights (w_is_bf16 = 0) or from bf16 weights each rounded to fp16 first (w_is_bf16 = 1):
 * s = fp16(max|w| / 7) per `group` weights of a row, q = clamp(rint(w / s), -8, 7) (0 where s == 0).
 * w [rows, cols] -> wq [rows, cols/8], ws [rows, cols/group]. group % 8 == 0, cols % group == 0, group <= 4096.
 * Replaces: quantize4 (llama/run.py:56-70) and the "q4" recipe line of llama/st2bin.c:44-66. */
int aq_quantize_q4(const uint16_t* w, int32_t w_is_bf16, int64_t rows, int64_t cols, int32_t group, uint32_t* wq,
                   uint16_t* ws);

/* Q4W from bf16 weights with the least-squared-error scale fp16(m / d), d = 6.5, 6.75, ..., 9 (first minimum wins).
 * group % 8 == 0, group <= 256. Replaces: the "q4" recipe line of qwen3moe/convert.c:120-159. */
int aq_quantize_q4_searched(const uint16_t* w_bf16, int64_t rows, int64_t cols, int32_t group, uint32_t* wq,
                            uint16_t* ws);

/* GGUF Q4_0 (18-byte blocks of 32: fp16 d, then 16 bytes, element j low nibble of byte j, j + 16 its high nibble)
 * -> Q4W words (nib ^ 8) and the fp16 scales unchanged (G = 32). cols % 32 == 0.
 * Replaces: q4_block / the "q4" recipe line of lfm2/convert.c:59-71. */
int aq_gguf_q4_0_to_q4w(const uint8_t* blocks, int64_t rows, int64_t cols, uint32_t* wq, uint16_t* ws);

/* GGUF Q4_0 -> fp16 [rows, cols]: (nib - 8) * d in fp32, rounded to fp16.
 * Replaces: q4_dequant + the "h4" recipe line of lfm2/convert.c:73-80. */
int aq_gguf_q4_0_to_f16(const uint8_t* blocks, int64_t rows, int64_t cols, uint16_t* out);

/* GGUF Q6_K (210-byte super-blocks of 256: ql[128] low nibbles, qh[64] high 2-bit pairs, int8 scales[16] one per 16
 * weights, fp16 d) -> Q6W: q [rows, cols/256, 208] (each super-block's first 208 bytes, unchanged) and d fp16
 * [rows, cols/256]. cols % 256 == 0. Replaces: the "q6" recipe line of lfm2/convert.c:148-155. */
int aq_gguf_q6_k_to_q6w(const uint8_t* blocks, int64_t rows, int64_t cols, uint8_t* q, uint16_t* d);

/* GGUF Q6_K -> fp16 [rows, cols]: (d * sc) * (q - 32) in fp32, rounded to fp16, where element 128 h + 32 j + l of a
 * super-block has q = (nibble j / 2 of ql[64 h + 32 (j % 2) + l]) | (bits 2 j, 2 j + 1 of qh[32 h + l]) << 4 and
 * sc = scales[8 h + 2 j + l / 16]. Replaces: q6_dequant + the "h6" recipe line of lfm2/convert.c:82-103,163-175. */
int aq_gguf_q6_k_to_f16(const uint8_t* blocks, int64_t rows, int64_t cols, uint16_t* out);

/* T2W scales from the (scale, bias) fp32 pairs [groups = K/128, n, 2] that bonsai/convert.cpp:44-61 (emitPacked)
 * writes beside the transposed codes (those are T2W words already): s fp16 [groups, n] = the scales. Returns
 * AQ_ERR_ARG, writing nothing, if any group is not ternary (bias != -scale) or a scale is not exact in fp16. */
int aq_t2w_scales_from_pairs(const float* params, int64_t groups, int64_t n, uint16_t* s);

/* MLX 2-bit projections -> one fused T2W matrix: part p has codes [rows[p], K/16], scales and biases fp16
 * [rows[p], K/128]; w [K/16, sum rows] (transposed), s [K/128, sum rows]. Returns AQ_ERR_ARG, writing nothing, if any
 * group is not ternary (bias != -scale). K % 128 == 0. Replaces: addPacked (qwen3/convert.cpp:39-74). */
int aq_t2w_from_mlx(const uint32_t* const* codes, const uint16_t* const* scales, const uint16_t* const* biases,
                    const int64_t* rows, int32_t parts, int64_t k, uint32_t* w, uint16_t* s);

#ifdef __cplusplus
}
#endif

#endif /* AQ_H */
