/*
 * fbsa.h -- C ABI of the MI355X (gfx950) block-pair selection + fused
 * block-sparse attention library (libfbsa.so).
 *
 * Every entry point is stateless and re-entrant, takes raw device pointers,
 * 64-bit sizes/strides in elements, and the HIP stream to launch on (passed as
 * void*, a hipStream_t; NULL = the default stream). Nothing here allocates
 * device memory: workspaces are sized by the *_workspace_bytes queries and
 * provided by the caller. Arguments are validated on the host before any
 * launch; a non-zero status is returned with a message in fbsa_last_error()
 * (thread-local). Launches are asynchronous.
 *
 * Tensor layouts (element strides; the innermost dimension D is contiguous):
 *   q, o, do, dq   (B, Hq, L, D)   strides {b, h, l}
 *   k, v, dk, dv   (B, Hkv, L, D)  strides {b, h, l}
 *   out_gate       (B, Hq, L, D)   strides {b, h, l} (e.g. Qwen's (B,L,Hq*D) view)
 *   sel, gate      (B, Hsel, nblk, kk) contiguous, int32 / fp32; Hsel = 1
 *                  (one selection shared by every head) or Hkv (per KV head)
 *   lse            (B, Hq, L) contiguous fp32
 *   (the backward's row statistics, delta and lse * log2 e, live in its
 *   workspace in an internal layout; only the stage functions read them)
 *
 * The reference (apoc/fused-block-sparse-attention) is Python + Triton; the
 * entry points below replace the device work behind its Python surfaces, as
 * cited on each declaration.
 */
#ifndef FBSA_H
#define FBSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of float tensors (q, k, v, o, do, dq, dk, dv, out_gate, pooled operands). */
enum { FBSA_F32 = 0, FBSA_BF16 = 1, FBSA_F16 = 2 };

/* Attention mask rules.
 * NONE         every key of every slot at a position < l_valid
 *              (src/triton_kernel.py:20-74 with CAUSAL=False; l_valid < L only
 *              for the padded non-causal dense path, src/qwen_blocksparse.py:37-41)
 * SLOT_CAUSAL  slot 0: key row <= query row; slot s>0 valid iff sel < i
 *              (src/triton_kernel.py:57-61; src/ssa_model.py:167-183)
 * TOKEN_CAUSAL key pos <= query pos, key pos < l_valid, first occurrence of the
 *              block index in the row (src/qwen_blocksparse.py:67-72) */
enum { FBSA_MASK_NONE = 0, FBSA_MASK_SLOT_CAUSAL = 1, FBSA_MASK_TOKEN_CAUSAL = 2 };

/* Status codes. */
enum { FBSA_OK = 0, FBSA_EINVAL = 1, FBSA_EUNSUPPORTED = 2, FBSA_EHIP = 3, FBSA_EWORKSPACE = 4 };

typedef struct fbsa_attn_desc {
  int32_t dtype;   /* FBSA_F32 / FBSA_BF16 / FBSA_F16 */
  int32_t mask;    /* FBSA_MASK_* */
  int64_t B, Hq, Hkv;
  int64_t L;       /* sequence length, a multiple of bs (nblk * bs) */
  int64_t D;       /* head dim: 32, 64, 128 or 256 */
  int64_t bs;      /* block size: 16, 32, 64 or 128 */
  int64_t nblk, kk;
  int64_t hsel;    /* 1 or Hkv */
  int64_t l_valid; /* positions >= l_valid are padding keys (NONE, TOKEN_CAUSAL) */
  float scale;     /* softmax scale applied to q.k before the gate bias */
  int32_t flags;   /* FBSA_FLAG_* bits (DENSE: forward and backward; OUT_GATE: backward only) */
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], sog[3];
} fbsa_attn_desc;

const char *fbsa_last_error(void);
int fbsa_version(void);

/* Fused block-sparse forward. o = softmax(scale*q.k^T + gate) v over the
 * selected key blocks (times sigmoid(out_gate) when out_gate != NULL);
 * lse (nullable) = natural-log normaliser of the un-gated softmax, summed in
 * fp32 from the unrounded exponentials for every input dtype (16-bit P enters
 * only the P.V product).
 * gate (nullable): fp32 additive bias per (b, hsel, i, slot).
 * Replaces _bsattn_fwd / bsattn_forward (src/triton_kernel.py:20-74, 184-207)
 * and the gather+SDPA of _gather_and_attend (src/ssa_model.py:57-90) and
 * blocksparse_forward (src/qwen_blocksparse.py:57-84). */
int fbsa_fwd(const fbsa_attn_desc *d, const void *q, const void *k, const void *v,
             const int32_t *sel, const float *gate, const void *out_gate,
             void *o, float *lse, void *stream);

/* The forward for query blocks [i_begin, i_end) only (O and LSE rows of those
 * blocks are written; sel rows outside the range are not read). Lets a caller
 * overlap the selection of later query blocks with the forward of earlier
 * ones on two streams. fbsa_fwd is the range [0, nblk). No counterpart in
 * the reference (its forward is one call over all blocks). */
int fbsa_fwd_rows(const fbsa_attn_desc *d, int64_t i_begin, int64_t i_end, const void *q, const void *k,
                  const void *v, const int32_t *sel, const float *gate, const void *out_gate, void *o,
                  float *lse, void *stream);

/* Dense causal per-block attention mass, the teacher SelectOracle selects from
 * (capture_mass, src/eval_qwen_ppl.py:65-108): mass (B, Hq, nblk, nblk) fp32,
 * entry (i, j) = the mean over block i's query rows t of the softmax
 * probability summed over block j's keys s <= t; zero above the diagonal (the
 * caller averages over each KV head's query heads, as the reference does).
 * Scores are rounded like torch's 16-bit matmul and scale multiply,
 * rnd(rnd(q.k) * scale); the softmax is fp32. Reads d->dtype (bf16 or f16),
 * B, Hq, Hkv, L = nblk * bs, D (64, 128, 256), bs (64, 128), nblk, scale, sq,
 * sk. ws: fbsa_block_mass_workspace_bytes(d) bytes, 16-byte aligned (the row
 * log-sum-exp). Replaces the per-query-block loop of capture_mass. */
size_t fbsa_block_mass_workspace_bytes(const fbsa_attn_desc *d);
int fbsa_block_mass(const fbsa_attn_desc *d, const void *q, const void *k, float *mass, void *ws, void *stream);

/* ---- selection ------------------------------------------------------- */

/* Pooling ops over each block of bs tokens (tokens >= l_valid read as 0).
 * MEAN_TOK_THEN_GRP  mean over tokens (rounded), then over the grp heads
 *                    (rounded): q.view(B,H,nblk,bs,D).mean(3).mean(1)
 *                    (src/ssa_model.py:287-288)
 * MEAN_GRP_THEN_TOK  mean over the grp heads (rounded), then tokens (rounded)
 *                    (src/qwen_blocksparse.py:113)
 * MAX / MIN          per-block max / min (src/ssa_model.py:117;
 *                    src/qwen_blocksparse.py:115-116)
 * MINMAX             min into out, max into out2 */
enum { FBSA_POOL_MEAN_TOK_THEN_GRP = 0, FBSA_POOL_MEAN_GRP_THEN_TOK = 1,
       FBSA_POOL_MAX = 2, FBSA_POOL_MIN = 3, FBSA_POOL_MINMAX = 4 };

typedef struct fbsa_pool_desc {
  int32_t dtype, op;
  int64_t B, H, L, D, bs, nblk, grp, l_valid;
  int64_t sx[3];   /* input strides {b, h, l}; output (B, H/grp, nblk, D) contiguous */
} fbsa_pool_desc;

int fbsa_pool(const fbsa_pool_desc *d, const void *x, void *out, void *out2, void *stream);

/* Score functions of the nblk x nblk pooled contraction (never stored):
 * DOT    rnd(a.b1)                                   (src/scale_sel.py:33-35)
 * MAX2   max(rnd(a.b1), rnd(a.b2))                   (src/ssa_model.py:118-119)
 * QUEST  rnd(rnd(relu(a).b1) + rnd(min(a,0).b2))     (src/qwen_blocksparse.py:117-120)
 * rnd() rounds the exact value to fp32 and then to the operand dtype. */
enum { FBSA_SCORE_DOT = 0, FBSA_SCORE_MAX2 = 1, FBSA_SCORE_QUEST = 2 };
/* OWN_FIRST:   sel = [i, top-k content blocks by descending score], own block
 *              excluded, future blocks excluded when causal, fills = i
 *              (src/ssa_model.py:151-165)
 * SORTED_SINK: _finish: top-k over j <= i (own included), non-finite picks
 *              -> i, + own (+ sink block 0), sorted ascending
 *              (src/qwen_blocksparse.py:87-99)
 * SORTED_TOPK: the top-k set of SORTED_SINK alone (non-finite picks -> i,
 *              ascending, no own or sink appended): the candidate stage
 *              cand = s1.topk(M) of SelectTwoStage, used as a set
 *              (src/qwen_blocksparse.py:289-290). fbsa_select_qmax only. */
enum { FBSA_SEL_OWN_FIRST = 0, FBSA_SEL_SORTED_SINK = 1, FBSA_SEL_SORTED_TOPK = 2 };

/* fbsa_select_desc.flags: bits 8..23 = candidate tiles (64 key blocks each)
 * per workgroup of the MFMA path, 0 = chosen from the sizes. Tuning and tests
 * only; the result does not depend on it. Other bits must be 0. */
enum { FBSA_SEL_CHUNK_SHIFT = 8 };

typedef struct fbsa_select_desc {
  int32_t dtype, score, convention, causal, sink, flags;
  int64_t B, H, nblk, D, topk, kk;  /* operands (B, H, nblk, D) contiguous */
} fbsa_select_desc;

/* Streaming score + top-k: writes sel (B,H,nblk,kk) int32 and, when sel_score
 * != NULL, the score of each chosen slot as fp32 (for the log-sigmoid gate).
 * Ties break towards the lower block index. Top-k budgets up to 62 run on
 * wave-wide lists; larger ones (up to 4096) on one workgroup per query row
 * with the row's keys in LDS (same scores, same result). With a workspace of at least
 * fbsa_select_workspace_bytes() bytes (16-byte aligned; nonzero for 16-bit
 * operands of dim >= 32) scores are formed on MFMA and verified exactly (fp64
 * only where the rounding is ambiguous); without one, every score is formed
 * in fp64. Both give the same result.
 * Replaces the topk selection of src/ssa_model.py:151-165,
 * src/bench_crossover.py:41-54 and SelectMax/_finish
 * (src/qwen_blocksparse.py:87-121). */
size_t fbsa_select_workspace_bytes(const fbsa_select_desc *d);
int fbsa_select(const fbsa_select_desc *d, const void *a, const void *b1, const void *b2,
                int32_t *sel, float *sel_score, void *workspace, size_t workspace_bytes,
                void *stream);

/* Selection for query blocks [row_begin, row_end) only (those rows of sel and
 * sel_score are written). Causal selections of a prefix of rows read only
 * that prefix of the operands. fbsa_select is the range [0, nblk). No
 * counterpart in the reference (it selects all rows at once). */
int fbsa_select_rows(const fbsa_select_desc *d, int64_t row_begin, int64_t row_end, const void *a,
                     const void *b1, const void *b2, int32_t *sel, float *sel_score, void *workspace,
                     size_t workspace_bytes, void *stream);

/* Mean-pooled q.k block selection in one call: pools q into qp and k into kp
 * (dq, dk: op MEAN_TOK_THEN_GRP; outputs (B, H/grp, nblk, D) contiguous, as
 * fbsa_pool writes them) and selects with score DOT over (qp, kp) as
 * fbsa_select with d. dq and dk share dtype, B, L, D, bs, nblk and l_valid,
 * and H/grp equals d->H for both. With a workspace of at least
 * fbsa_select_workspace_bytes(d) bytes and 16-bit operands of dim 32 or 64
 * (top-k budget <= 32), both tensors are pooled by one launch that also writes
 * the selection's row norms, so the call takes three launches instead of five;
 * otherwise it runs fbsa_pool twice and fbsa_select. qp, kp, sel and sel_score
 * are identical either way. Replaces the pooling of src/ssa_model.py:287-288
 * (and src/bench_crossover.py:41-45), the score qpool.kpool^T of
 * src/scale_sel.py:33 and the top-k of src/ssa_model.py:151-165. */
int fbsa_select_mean_pooled(const fbsa_pool_desc *dq, const void *q, void *qp, const fbsa_pool_desc *dk,
                            const void *k, void *kp, const fbsa_select_desc *d, int32_t *sel,
                            float *sel_score, void *workspace, size_t workspace_bytes, void *stream);

/* fbsa_select without a workspace argument and without any allocation, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The MFMA selection's workspace comes from a static device array
 * of FBSA_SELECT_SCRATCH_BYTES bytes that every GPU the library runs on holds
 * until the process ends; the current device's array is used (the stream
 * must belong to that device). A selection needing more
 * (fbsa_select_workspace_bytes() > FBSA_SELECT_SCRATCH_BYTES) is rejected with
 * FBSA_EWORKSPACE before any launch. All calls on one GPU share its array:
 * calls that overlap on one GPU (two streams or threads) race. Results equal
 * fbsa_select's. */
#define FBSA_SELECT_SCRATCH_BYTES (32u << 20)
int fbsa_select_noalloc(const fbsa_select_desc *d, const void *a, const void *b1, const void *b2,
                        int32_t *sel, float *sel_score, void *stream);

/* Row-block max Quest selection. The score of query block i and key block j
 * is the best Quest score over the tok query vectors of block i:
 *   score(i, j) = max_t rnd(rnd(relu(a_t).b1_j) + rnd(min(a_t,0).b2_j))
 * (b1 = per-block key max, b2 = key min; rnd as for FBSA_SCORE_QUEST), over
 * the key blocks j <= i or, when cand != NULL, over row i's entries of cand
 * (B,H,nblk,ncand) int32 (each row ascending, as SORTED_TOPK writes it;
 * repeats and entries outside [0, i] are skipped). Then the top-k of the
 * convention (SORTED_SINK or SORTED_TOPK), ties to the lower block index.
 * a: (B,H,la,D) contiguous query vectors, block i = vectors [i*tok,
 * (i+1)*tok), vectors at or past la are zero (the reference's zero padding);
 * b1, b2: (B,H,nblk,D) contiguous; sel: (B,H,nblk,kk). Operands are finite.
 * 16-bit operands with tok 64 or 128, D >= 64 and a workspace of at least
 * fbsa_select_qmax_workspace_bytes() bytes (16-byte aligned; it holds the
 * key-block norms) bracket the scores on MFMA and compute exactly (float64)
 * only the scores the top-k needs; other cases, no workspace, or
 * FBSA_QMAX_EXACT compute every score in float64; all give the same result. Supports D in {32,64,128,256}, nblk <= 65536 and at most 8192
 * columns per row (nblk, or ncand with a candidate list). Replaces
 * SelectMaxQMax.select (tok = bs, a = the GQA-group mean of every token;
 * src/qwen_blocksparse.py:216-241) and both stages of SelectTwoStage
 * (tok = 1 on the pooled query for the candidates, then tok = bs over them;
 * src/qwen_blocksparse.py:267-299). */
enum { FBSA_QMAX_EXACT = 1 };

typedef struct fbsa_qmax_desc {
  int32_t dtype, convention, sink, flags;
  int64_t B, H, nblk, D, tok, la, topk, kk, ncand;
} fbsa_qmax_desc;

size_t fbsa_select_qmax_workspace_bytes(const fbsa_qmax_desc *d);
int fbsa_select_qmax(const fbsa_qmax_desc *d, const void *a, const void *b1, const void *b2,
                     const int32_t *cand, int32_t *sel, void *workspace, size_t workspace_bytes,
                     void *stream);

/* ---- backward -------------------------------------------------------- */

/* fbsa_attn_desc.flags bits. OUT_GATE: the backward will be given out_gate
 * (the forward applied o <- o * sigmoid(out_gate)); the workspace then also
 * holds the gate-scaled upstream gradient.
 * DENSE (forward and backward): every key block is selected, slot s holding
 * block s (kk must equal nblk); sel is not read (may be NULL) and gate must be
 * NULL. With FBSA_MASK_TOKEN_CAUSAL query block i reads blocks 0..i (causal
 * dense attention), with FBSA_MASK_NONE every block; keys at or past l_valid
 * are padding in both. The block list is implicit, so the forward takes any
 * length, and the backward's transposed lists need no sort (their total,
 * B * hsel * the number of (query block, key block) pairs, must stay below
 * 2^31). Replaces the SDPA fast path of blocksparse_forward
 * (src/qwen_blocksparse.py:37-41).
 * DGATE (backward): the gate gradient will be asked for (dgate != NULL); the
 * workspace then also holds each query row's probability mass per slot
 * (B*Hq*L*kk fp32), with which a 16-bit gate gradient is corrected to the
 * row's fp32 delta. Required with dgate for 16-bit types. */
enum { FBSA_FLAG_OUT_GATE = 1, FBSA_FLAG_DENSE = 2, FBSA_FLAG_DGATE = 4 };

/* Workspace for the backward stages below (one opaque region, 256-byte
 * aligned): per-row softmax statistics, the block-transposed index (CSR of
 * the valid (query block, slot) pairs per key block, sorted by a stable radix
 * sort so the dK/dV summation order is fixed), per-head gate-gradient
 * partials and, with FBSA_FLAG_OUT_GATE, the gate-scaled dO.
 * Returns 0 (with fbsa_last_error set) when the descriptor is invalid. */
size_t fbsa_bwd_workspace_bytes(const fbsa_attn_desc *d);

/* Stage 1. Row statistics: delta[b,h,t] = sum_d dout*o and lse*log2(e) into
 * the workspace. With out_gate (FBSA_FLAG_OUT_GATE): dout_gate = dout*o*
 * (1 - sigmoid(out_gate)) (B,Hq,L,D contiguous) and the workspace copy
 * dout*sigmoid(out_gate) used by the later stages. o, dout strides: so, sdo. */
int fbsa_bwd_prep(const fbsa_attn_desc *d, const void *o, const void *dout, const float *lse,
                  const void *out_gate, void *dout_gate, void *workspace, size_t workspace_bytes,
                  void *stream);

/* Stage 2. Block-transposed index of sel: for each (b, hsel, key block j) the
 * valid (i, slot) pairs that read it, ascending (deterministic CSR). */
int fbsa_transpose_index(const fbsa_attn_desc *d, const int32_t *sel, void *workspace,
                         size_t workspace_bytes, void *stream);

/* Stage 3. dq (B,Hq,L,D contiguous) over each query block's selected key
 * blocks; when dgate != NULL also the fp32 gate gradient (B,Hsel,nblk,kk),
 * summed over the heads sharing a selection in a fixed order (0 for masked
 * slots). Needs stage 1. For 16-bit types it also replaces each row's delta in
 * the workspace by sum P*dP over the row's keys, accumulated in fp32 from the
 * unrounded P (the reference's D, src/triton_kernel.py:132-150); the gate
 * gradient uses that delta. */
int fbsa_bwd_dq(const fbsa_attn_desc *d, const void *q, const void *k, const void *v,
                const void *dout, const int32_t *sel, const float *gate, void *dq, float *dgate,
                void *workspace, size_t workspace_bytes, void *stream);

/* Stage 4. dk, dv (B,Hkv,L,D contiguous), one workgroup per key block walking
 * its transposed list (and the GQA group's query heads) in order: no atomics,
 * bitwise repeatable. Needs stages 1 and 2, and stage 3 for the fp32-exact
 * delta of 16-bit types (without it the prep's estimate from the stored O is
 * used). */
int fbsa_bwd_dkdv(const fbsa_attn_desc *d, const void *q, const void *k, const void *v,
                  const void *dout, const float *gate, void *dk, void *dv, void *workspace,
                  size_t workspace_bytes, void *stream);

/* All four stages in order. lse is the forward's (fbsa_fwd) output; o is the
 * forward output (gated when out_gate != NULL). dgate and dout_gate are
 * nullable. For bf16 without an output gate the prep stage's only
 * output is the row statistics, and the dQ stage forms them itself from o and
 * lse (the same values, summed in the same order), so no separate pass over o
 * and dout runs, and the index stage (which reads sel alone) runs beside the
 * dQ stage on a second stream (one per host thread and device, created on
 * first use with the default priority), joined by an event before dK/dV (under
 * stream capture all stages run in order on `stream`); work on `stream` after
 * the call is ordered after all of it. Replaces _bsattn_bwd / bsattn_backward
 * (src/triton_kernel.py:77-181, 210-234) and the autograd of the gather path
 * (src/ssa_model.py:57-90). */
int fbsa_bwd(const fbsa_attn_desc *d, const void *q, const void *k, const void *v, const void *o,
             const void *dout, const float *lse, const int32_t *sel, const float *gate,
             const void *out_gate, void *dq, void *dk, void *dv, float *dgate, void *dout_gate,
             void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FBSA_H */
