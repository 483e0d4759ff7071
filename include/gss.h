/*
 * gss.h — C ABI of the MI355X (gfx950) self-speculative round kernels.
 *
 * Every entry point takes raw device pointers, explicit sizes and a HIP stream (passed as an opaque pointer, the
 * value of hipStream_t), enqueues its kernels on that stream and returns a status code; nothing synchronises and
 * nothing allocates. The caller owns every buffer. Lengths that change from round to round (committed KV length,
 * accept length) are read from device memory, so a sequence of calls can be captured into a HIP graph and replayed.
 *
 * Tensor layouts (bf16 = 16-bit brain float, stored as its bit pattern):
 *   q            [bs, W, Hq, D]                   window queries, already rotated
 *   k_pages      [n_pages, Hkv, page, D]          paged K cache (one layer)
 *   v_pages      [n_pages, Hkv, D, page]          paged V cache (one layer), token index fastest within a page
 *   page_table   int32 [bs, pt_stride]            page ids of each sequence, in position order
 *   k_win, v_win [bs, W, Hkv, D]                  the window's own K/V (staging, not yet in the cache)
 *   logits       [bs, W, V] (row stride ld_row elements), bf16 or fp32
 *
 * Greedy rule shared with the reference: index of the row maximum, lowest index on exact ties, NaN counts as max.
 */
#ifndef GSS_H
#define GSS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* gss_stream_t; /* a hipStream_t; NULL = the default stream */

enum gss_status {
  GSS_OK = 0,
  GSS_ERR_ARG = 1,         /* a size, stride or pointer is invalid */
  GSS_ERR_UNSUPPORTED = 2, /* a shape the kernels are not built for (head_dim, page size, window, group) */
  GSS_ERR_WORKSPACE = 3,   /* workspace missing or smaller than the size query returned */
  GSS_ERR_LAUNCH = 4       /* the HIP launch itself failed */
};

enum gss_dtype { GSS_BF16 = 0, GSS_F32 = 1 };

/* argmax rule flags (gss_argmax_accept) */
enum gss_argmax_flags {
  /* argmax(softmax(float(logits))) as src/models/glm_ocr_dllm.py:997-1002 computes it: a row holding a NaN or +inf
   * has an all-NaN fp32 softmax, whose argmax is 0. Without the flag a NaN counts as the maximum (torch.argmax on
   * the raw logits, the serving worker's rule: selfspec_diffusion_worker.py:742). */
  GSS_ARGMAX_SOFTMAX = 1,
  /* with GSS_ARGMAX_SOFTMAX: the last row of each sequence keeps the raw rule (natcache's verify takes ar_pred from
   * the softmax and the bonus from the raw logits of the last row, src/fast_sampling.py:572-575) */
  GSS_ARGMAX_LAST_RAW = 2
};

const char* gss_version(void);
const char* gss_status_string(int status);

/* ---------------------------------------------------------------- (a)/(b) attention over paged KV + window ---
 * Replaces the draft/verify attention of the self-spec forwards: the flashinfer paged prefill the SGLang hooks
 * route by role (patches/sglang/sglang_0.5.10_selfspec.patch:486-522; planner
 * patches/sglang/python/sglang/srt/speculative/selfspec_fast_attn.py:168-465) and the flex-attention masks of the
 * in-process drop-in (src/fast_sampling.py:508-514).
 *
 * Query row w of sequence b attends to the committed prefix, keys [0, L) with L = prefix_len[b] + prefix_extra,
 * read from the pages, and to window keys from k_win/v_win:
 *   draft  (gss_draft_attn):  rows w < n_causal see window rows 0..w; rows w >= n_causal see all W window rows.
 *                             n_causal = 1 is the serving draft [x0 | MASK x B] and natcache rounds >= 1;
 *                             n_causal = 0 is natcache round 0 and the block-diffusion sampler's full block.
 *   verify (gss_verify_attn): row w sees window rows 0..w (causal, bottom-right aligned).
 * scale multiplies q.k (1/sqrt(D) for GLM). Supported: D in {64, 128}, page = 16, 1 <= W <= 64, Hq % Hkv == 0.
 *
 * The plan (caller-owned, no process-wide state): the kernel and the key partition, 64-token tiles by absolute
 * position, tiles_per_split of them per split. It fixes the order in which every key is combined, so any two calls
 * with the same plan compute a query row the same way whatever W, L or the rest of the batch: a verify row equals
 * the AR step of the same token bit for bit, and a sequence decoded alone with its batch's plan reproduces its rows
 * of the batched decode bit for bit. Keep one plan while a cache is decoded. L is clamped to
 * min(plan->max_kv_len, pt_stride * page): keys past the plan's capacity are never read (callers keep every
 * prefix within it; the splits cover max_kv_len plus a full window of 64). No counterpart in the reference: the
 * flashinfer planner's split-KV choice (selfspec_fast_attn.py:288-332) is internal to flashinfer.
 */
enum gss_attn_kernel {
  GSS_ATTN_ROWGROUP = 0, /* the rows of a split over up to ceil(R / 48) workgroups: fills the chip from few splits */
  GSS_ATTN_WIDE = 1      /* one workgroup per key split for all rows, tiles through a ring of LDS slots */
};

typedef struct gss_attn_plan {
  int kernel;          /* gss_attn_kernel */
  int tiles_per_split; /* 1..256 */
  int n_split;         /* 1..256 splits; n_split * tiles_per_split * 64 >= max_kv_len + 64 */
  int max_kv_len;      /* capacity: the longest prefix L a call may see */
} gss_attn_plan;

/* Fill *plan for a batch of bs sequences: about target_wgs / (bs * Hkv) key splits per sequence and kv head, each
 * at least min_tiles tiles; the wide kernel when bs * Hkv >= wide_min. Zero takes the default (896, 4, 16). */
int gss_attn_make_plan(int bs, int Hkv, int max_kv_len, int target_wgs, int min_tiles, int wide_min,
                       gss_attn_plan* plan);

/* Workspace bytes (split partials; no zeroing needed) of a call with this shape and plan. */
int gss_attn_workspace_size(int bs, int Hq, int Hkv, int D, int W, const gss_attn_plan* plan, size_t* bytes);

int gss_draft_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table, int pt_stride,
                   const int32_t* prefix_len, int prefix_extra, const void* k_win, const void* v_win, void* out,
                   int bs, int W, int n_causal, int Hq, int Hkv, int D, int page, float scale,
                   const gss_attn_plan* plan, void* workspace, size_t workspace_bytes, gss_stream_t stream);

int gss_verify_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                    int pt_stride, const int32_t* prefix_len, int prefix_extra, const void* k_win, const void* v_win,
                    void* out, int bs, int W, int Hq, int Hkv, int D, int page, float scale,
                    const gss_attn_plan* plan, void* workspace, size_t workspace_bytes, gss_stream_t stream);

/* ---------------------------------------------------------------- (c) argmax + accept + bonus -------------------
 * Replaces torch.argmax over the verify/draft logits (selfspec_diffusion_worker.py:742; src/fast_sampling.py:545,
 * :574-575) and sgl-kernel verify_tree_greedy on the worker's linear chain (selfspec_fast_commit.py:150-160,
 * chain layout selfspec_diffusion_worker.py:530-548).
 *
 * target[b, r] = argmax of logits row (b, r), r in [0, W): the maximum, the lowest index on ties; flags selects
 * the rule for rows with a NaN or +inf (gss_argmax_flags).
 * With window != NULL (the verify ids [a0, d_1..d_{W-1}] of each sequence) also:
 *   accept_len[b] = number of leading r in [0, W-2] with target[b, r] == window[b, r+1]
 *   next_x0[b]    = target[b, accept_len[b]]              (the correction, or the bonus when all W-1 matched)
 *   packed[b]     = (window[b,0], accept_len[b], target[b,0..W-1] with entries past accept_len zeroed)
 *                   the row layout of _ss_commit_kernel's readback (selfspec_fast_commit.py:125-138); may be NULL.
 * Workspace: gss_argmax_workspace_size bytes, zeroed once after allocation. Its first 1152 KiB are arrival counters
 * (nine 128-byte lines per sequence) at a fixed offset, so one workspace serves calls with different bs, W, V (sized
 * for the largest). bs <= 1024, W <= 64, V <= 131072.
 */
int gss_argmax_workspace_size(int bs, int W, int V, size_t* bytes);

int gss_argmax_accept(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int flags,
                      const int32_t* window, int32_t* target, int32_t* accept_len, int32_t* next_x0, int32_t* packed,
                      void* workspace, size_t workspace_bytes, gss_stream_t stream);

/* gss_argmax_accept_noalloc: gss_argmax_accept (same arguments and outputs, bit for bit) with no workspace argument
 * and no allocation of any kind. No counterpart in the reference: it is for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Its scratch (arrival counters and chunk
 * winners, 1,122,304 bytes) is a device array inside the library: each GPU the library runs on holds one copy
 * until the process ends, set up on the first call on that device (the current device). Limits: bs <= 64,
 * W <= 64, V <= 131072 (GSS_ERR_UNSUPPORTED beyond them). Every call on one GPU shares that GPU's scratch: calls
 * that overlap on one GPU (different streams, or host threads) race; calls ordered on one stream do not. */
int gss_argmax_accept_noalloc(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int flags,
                              const int32_t* window, int32_t* target, int32_t* accept_len, int32_t* next_x0,
                              int32_t* packed, gss_stream_t stream);

/* ---------------------------------------------------------------- block-diffusion unmask step -------------------
 * Replaces one iteration of the threshold-unmask loop of the cached block-diffusion decode at temperature 0
 * (src/fast_sampling.py:206-216 generate_cached; src/fast_sampling_batched.py:198-211 generate_cached_batched):
 *   logits  = lm_head rows of the block forward, [bs, W, V] (row stride ld_row)
 *   shifted = in-block token shift: position j reads row max(j - 1, 0)
 *   x1[j]   = argmax of softmax(float(shifted[j])) (GSS_ARGMAX_SOFTMAX rule), conf[j] = its probability
 *   unmask  = masked positions (block == mask_id) with conf > threshold, plus the first position of the largest
 *             conf among the masked ones (NaN as the largest); block[j] = x1[j] where unmasked.
 * Outputs (each may be NULL): x1 and conf [bs, W] (every position, masked or not), n_unmasked[b] (positions the rule
 * unmasked), n_left[b] (positions holding mask_id afterwards), seed[b] = argmax of row W - 1 without shift (the next block's seed after the commit forward,
 * src/fast_sampling.py:187-190). A block without masks is left unchanged. conf is 1 / sum(exp(x - max)), summed in
 * a fixed order (within a few ulp of torch's softmax).
 * Workspace: gss_unmask_workspace_size bytes, zeroed once after allocation (the first 1152 KiB are counters, the
 * same layout and limits as the argmax workspace).
 */
int gss_unmask_workspace_size(int bs, int W, int V, size_t* bytes);

int gss_unmask_step(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int32_t* block, int mask_id,
                    float threshold, int32_t* x1, float* conf, int32_t* n_unmasked, int32_t* n_left, int32_t* seed,
                    void* workspace, size_t workspace_bytes, gss_stream_t stream);

/* ---------------------------------------------------------------- (d) KV commit ---------------------------------
 * Replaces the commit half of _ss_commit_kernel (selfspec_fast_commit.py:139-147: seq_lens += acc + 1, rejected
 * slots released) and the natcache cache truncation (src/fast_sampling.py:600-605): the first n_b rows of the
 * window K/V of every layer are written into the pages at positions seq_lens[b] + j, j < n_b, and
 * seq_lens[b] += n_b, with n_b = (n_rows ? n_rows[b] : 0) + n_add. Rows >= n_b are discarded in place (never
 * written; the staging is overwritten by the next forward). slots (optional, [bs, W]) receives the slot index
 * page_table[b][pos / page] * page + pos % page of each committed row, -1 for the rest.
 * Window/page tensors of layer l start at k_win + l * win_layer_stride (elements), k_pages + l * page_layer_stride.
 * page must be 16 and Hkv * 16 * (D + 2) * 2 bytes at most 64 KiB (GSS_ERR_UNSUPPORTED otherwise).
 * Workspace: gss_kv_commit_workspace_size bytes (per-sequence counters), zeroed once after allocation.
 */
int gss_kv_commit_workspace_size(int bs, size_t* bytes);

int gss_kv_commit(const void* k_win, const void* v_win, int64_t win_layer_stride, void* k_pages, void* v_pages,
                  int64_t page_layer_stride, const int32_t* page_table, int pt_stride, int32_t* seq_lens,
                  const int32_t* n_rows, int n_add, int32_t* slots, int bs, int W, int n_layers, int Hkv, int D,
                  int page, void* workspace, size_t workspace_bytes, gss_stream_t stream);

/* ---------------------------------------------------------------- sampled verify (non-greedy requests) ---------
 * The serving round for requests that sample (selfspec_fast_commit.py:150-230, selfspec_sampling.py:139-293):
 * gss_penalize_rows gives every verify row the logits processing AR decode gives the same prefix, gss_sample_rows
 * draws a0 from the draft's causal row (sample mode) or runs speculative sampling of the draft chain against AR's
 * target distribution (verify mode). Logits are fp32 rows: row b * K + r at logits + (b * K + r) * ld_row.
 *
 * gss_penalize_rows (penalize_rows, selfspec_sampling.py:139-198, then logit_bias, selfspec_fast_commit.py:190-191),
 * in place: row r of sequence b sees the cumulated state of the committed tokens plus its in-block tokens
 * cand[b, 1..r]; the penalizers run in pen->order (the orchestrator's order): repetition (the penalty at those tokens
 * set to rep_pen[b]; positive logits divided, others multiplied), presence (set, subtracted), frequency (one
 * freq_pen[b] added per occurrence, subtracted), min_new_tokens (stop_pen[b] added while len_out[b] + r <
 * min_new[b]); logit_bias[b] (optional) is added last. State arrays are [bs, V] fp32, parameters [bs]. K <= 64.
 */
enum gss_penalizer { GSS_PEN_REPETITION = 1, GSS_PEN_PRESENCE = 2, GSS_PEN_FREQUENCY = 3, GSS_PEN_MIN_NEW_TOKENS = 4 };

typedef struct gss_penalties {
  int n_order;  /* penalizers in order[0..n_order) (gss_penalizer values, each at most once) */
  int order[4];
  const float* rep_cum;
  const float* rep_pen;
  const float* pres_cum;
  const float* pres_pen;
  const float* freq_cum;
  const float* freq_pen;
  const int32_t* len_out;
  const int32_t* min_new;
  const float* stop_pen;
  const float* logit_bias; /* or NULL */
} gss_penalties;

int gss_penalize_rows(float* logits, int64_t ld_row, int bs, int K, int V, const int32_t* cand,
                      const gss_penalties* pen, gss_stream_t stream);

/* gss_apply_vocab_mask: a grammar's vocabulary mask on logit rows (the grammar backend's apply_vocab_mask, which the
 * reference calls between the penalties and logit_bias, selfspec_fast_commit.py:186-189; the rows' masks come from
 * the host walk of fulldraft_bitmask, selfspec_sampling.py:305-337): logits[r * ld_row + v] = -inf where bit v % 32
 * of mask[r * ld_mask + v / 32] is clear (a set bit allows the token: the packed int32 layout of the grammar
 * backends' bitmasks). rows <= 65535, ld_mask >= ceil(V / 32). */
int gss_apply_vocab_mask(float* logits, int64_t ld_row, int rows, int V, const int32_t* mask, int64_t ld_mask,
                         gss_stream_t stream);

/* gss_sample_rows: target distribution of every row (verify_target_probs, selfspec_sampling.py:266-286): softmax of
 * logits / temperature[b] (temperature <= 0: a point mass at the row maximum), then filter 0 (none), 1 (flashinfer's
 * joint top-k / top-p: token q kept iff #{p > p_q} < top_k[b] and sum{p > p_q} < top_p[b], top_p >= 1 keeping
 * all; selfspec_sampling.py:230-244) or 2 (the pytorch backend: rank < top_k, mass before <= top_p, p >= max(p) *
 * min_p[b]; selfspec_sampling.py:253-263; tied values are kept or dropped together except the top-1 cut, which keeps
 * the lowest index) or 3 (the flashinfer backend in a batch that needs min_p, selfspec_sampling.py:276-281: tokens
 * with #{p > p_q} < top_k[b], renormalized; of those, tokens whose strictly greater renormalized mass is below
 * top_p[b] (top_p >= 1 keeps all); then p >= max(p) * min_p[b] when min_p is given and min_p[b] > 0),
 * renormalized; top_k <= 0 means no top-k cut. A draw with uniform u is the smallest token whose
 * prefix sum (index order) exceeds u * total.
 * Sample mode (cand NULL): sampled[b, r] = a draw from row (b, r) with uniforms[b * K + r] (a0 from the draft's
 * causal row: K = 1, ld_row = the stride between the sequences' rows).
 * Verify mode (cand = [bs, K] verify ids [a0, d_1..d_{K-1}], coins [bs, K] in (0, 1], uniforms [bs]): sgl-kernel
 * tree_speculative_sampling_target_only on the chain with a point-mass draft and thresholds 1
 * (selfspec_fast_commit.py:197-230): row j accepts d_{j+1} iff coins[b, j] <= p_j(d_{j+1}); accept_len[b] = the
 * first rejected row (K-1 when none); the committed targets are d_1..d_acc and then a draw from row acc without
 * d_{acc+1} (without removal when acc = K-1, the bonus), written to target[b, 0..acc] (rows past acc: that row's
 * own draw), next_x0[b] and packed[b] = (a0, acc, targets, zeros) as gss_argmax_accept writes them.
 * sampled[b, j] = row j's draw without its draft token. Workspace (verify mode): gss_sample_workspace_size bytes,
 * zeroed once. V <= 65536, K <= 64. */
int gss_sample_workspace_size(int bs, int K, size_t* bytes);

int gss_sample_rows(const float* logits, int64_t ld_row, int bs, int K, int V, int filter, const float* temperature,
                    const int32_t* top_k, const float* top_p, const float* min_p, const int32_t* cand,
                    const float* coins, const float* uniforms, int32_t* sampled, int32_t* target,
                    int32_t* accept_len, int32_t* next_x0, int32_t* packed, void* workspace, size_t workspace_bytes,
                    gss_stream_t stream);

/* ---------------------------------------------------------------- skinny GEMMs (decode projections) ----------
 * The dense projections of the decoder layer and the LM head (transformers GlmOcrTextAttention q/k/v/o_proj,
 * GlmOcrTextMLP gate_up/down_proj and lm_head, which the reference runs as torch linears through
 * src/fast_sampling.py:89-102). Y[M, N] = X[M, Kd] . W[N, Kd]^T, bf16 operands (row strides in elements, 16-byte
 * aligned), fp32 accumulation, M <= 65536, Kd % 32 == 0, N % 16 == 0. A row's result does not depend on M or on the
 * row's position (batch invariant), so speculative verify rows reproduce AR rows bit for bit, at every batch size.
 * The launch shape (waves per workgroup, k splits, features per workgroup) is a function of (N, Kd) and the
 * device's CU count only: it is the reduction order, so it is not a setting. The fused prologue and the post-norm
 * epilogue need every row in one workgroup: M <= 64 with either (GSS_ERR_UNSUPPORTED above).
 * gss_gemm: Y bf16 or fp32. gss_gemm_swiglu: W = gate_up with gate/up rows interleaved (2i = gate_i, 2i+1 = up_i),
 * act[M, F] = up * silu(gate). gss_gemm_rope_stage: W = [Wq; Wk; Wv], output q [bs, W, Hq, D] rotated,
 * window K/V [bs, W, Hkv, D] with K rotated (positions as gss_rope_stage with pos_offset 0).
 */
/* Optional fused prologue of the three GEMMs below (the GLM sandwich norm between sub-layers, GlmOcrTextDecoderLayer):
 *   h' = h_in + rmsnorm(a) * w_post   (a == NULL: h' = h_in),   x = rmsnorm(h') * w_next,   Y = x . W^T
 * with gss_add_rmsnorm's arithmetic (bit-identical to the unfused pair). Workgroup 0 stores h' to h_out (NULL: not
 * stored; must not alias h_in). Rows are Kd wide; needs Kd % 512 == 0 and Kd <= 1536. With pro == NULL the GEMM reads
 * x/ldx directly. */
typedef struct gss_norm_prologue {
  const void* a;      /* bf16 [M, Kd] or NULL */
  const void* h_in;   /* bf16 [M, Kd] residual stream */
  void* h_out;        /* bf16 [M, Kd] or NULL */
  const void* w_post; /* bf16 [Kd], used with a */
  const void* w_next; /* bf16 [Kd] */
  float eps;
  const float* a_parts; /* instead of a: fp32 partial sums [n_parts][M][Kd] from gss_gemm_parts (a = bf16 of their
                           sum in part order, as gss_add_rmsnorm_parts computes it), or NULL */
  int n_parts;
} gss_norm_prologue;

/* Norm epilogue of gss_gemm (the sandwich norm after o_proj and after the MLP down projection,
 * modeling_glm_ocr.py:263-310): once Y = X W^T is written (bf16, ldy == N, N = hidden size), every row gets
 *   h = h + rmsnorm(Y) * w_post;   x = rmsnorm(h) * w_next
 * with the arithmetic of gss_add_rmsnorm (bit-identical results). h is updated in place. Needs N % 512 == 0,
 * N <= 2048 and 16-byte aligned y, h, x and weights. The last workgroup to finish runs the norm. */
typedef struct gss_norm_epilogue {
  const void* w_post;
  void* h;
  const void* w_next;
  void* x;
  float eps;
} gss_norm_epilogue;

/* Workspace of the three GEMMs: per-column-tile counters at a fixed offset (zero them once after allocation; the
 * kernels leave them at zero) and the split-K partials of shapes whose column tiles alone would leave most CUs idle
 * (the k split depends on N and Kd only, never on M, so results stay batch invariant). Calls with M > 64 fold their
 * splits inside the kernel and need the counters block only, so the size stops growing at M = 64. One workspace
 * sized for the largest (M, N, Kd) serves every call on a stream. */
int gss_gemm_workspace_size(int M, int N, int Kd, size_t* bytes);

int gss_gemm(const void* x, int64_t ldx, const gss_norm_prologue* pro, const void* w, int64_t ldw, void* y,
             int64_t ldy, int M, int N, int Kd, int out_dtype, const gss_norm_epilogue* post, void* workspace,
             size_t workspace_bytes, gss_stream_t stream);

/* gss_gemm_parts: Y = X W^T (the torch bf16 linear of o_proj / down_proj) left as n_parts fp32 partial sums over
 * disjoint k ranges, parts [n_parts][M][N] (16-byte aligned); Y = bf16(parts[0] + parts[1] + ...) in part order,
 * which gss_add_rmsnorm_parts and the a_parts prologue compute. The k splits spread a projection with few column
 * tiles over twice the CUs without a handoff between them (the next kernel does the sum). n_parts =
 * gss_gemm_parts_count(N, Kd), a function of the weight shape (and the device's CU count) only: every M uses the
 * same partition, so rows stay batch invariant. No counterpart in the reference (how its linear is computed). */
int gss_gemm_parts_count(int N, int Kd, int* n_parts);

int gss_gemm_parts(const void* x, int64_t ldx, const void* w, int64_t ldw, float* parts, int M, int N, int Kd,
                   gss_stream_t stream);

int gss_gemm_swiglu(const void* x, int64_t ldx, const gss_norm_prologue* pro, const void* w_gu_interleaved,
                    int64_t ldw, void* act, int M, int F, int Kd, void* workspace, size_t workspace_bytes,
                    gss_stream_t stream);

int gss_gemm_rope_stage(const void* x, int64_t ldx, const gss_norm_prologue* pro, const void* w_qkv, int64_t ldw,
                        const int32_t* seq_lens, const int32_t* pos_delta, const float* inv_freq, int rot_dim,
                        void* q, void* k_win, void* v_win, int bs, int W, int Hq, int Hkv, int D, int Kd,
                        void* workspace, size_t workspace_bytes, gss_stream_t stream);

/* ---------------------------------------------------------------- serving-boundary bookkeeping ------------------
 * Integer steps of the SGLang round, in SGLang's buffer types, for a serving integration that keeps the pool's own
 * request / slot layout. One wavefront per sequence; no workspace.
 *
 * gss_ss_commit replaces _ss_commit_kernel (patches/sglang/python/sglang/srt/speculative/selfspec_fast_commit.py:
 * 108-147) and the cut rule of the host commit (selfspec_commit_rules.py:94-103, applied per request on the host
 * there). For row i with a = accept_len[i] (clamped into [0, K-1]) and T = [a0, t_0 .. t_a]:
 *   packed[i]        = (int32(a0[i * a0_stride]), a, predict[i*K .. i*K+K-1] with entries past a zeroed)
 *   out[i]           = predict[i*K + a];  seeds[req_pool_indices[i]] = out[i]  (rows whose pool index is outside
 *                      [0, n_seeds) leave the pool untouched)
 *   j                = the cut index: T[:j + 1] is committed. Without a finish rule (finish == NULL) or for a row
 *                      with budget[i] < 0 (a request whose finish needs the per-token path: grammar, stop strings),
 *                      j = a + 1. Otherwise j = the first t < lim with T[t] in stop_ids[i, :] or T[t] > vocab[i] or
 *                      T[t] < 0, else lim = min(a + 1, max(budget[i] - 1, 0)): where appending T one token at a time
 *                      with SGLang's length / stop-token / vocabulary checks would stop.
 *   cut[i] = j (cut may be NULL);  seq_lens[i] += j  (the verify rows 0 .. j-1 keep their KV)
 *   free_slots       = the slots of rows j .. K-1 that lie in pages holding no kept token (page: the KV page size;
 *                      slots are page-aligned, slot % page == position % page), every row's in row order, compacted;
 *                      *n_free = their count (n_free may be NULL). With page = 1 and no finish rule this is the
 *                      reference kernel's list: loc[i*K + a+1 .. i*K + K-1] of every row (sum(K-1-a) entries).
 * One wavefront per sequence; K <= 64; stop_ids [bs, n_stop] (negative entries are padding).
 */
typedef struct gss_finish_rule {
  const int32_t* budget;   /* [bs] max_new_tokens - len(output_ids); < 0: the per-token path decides (j = a + 1) */
  const int32_t* stop_ids; /* [bs, n_stop] */
  int n_stop;
  const int32_t* vocab;    /* [bs] the vocabulary bound of each request */
} gss_finish_rule;

int gss_ss_commit(const int32_t* predict, const int32_t* accept_len, const int64_t* a0, int64_t a0_stride,
                  const int64_t* req_pool_indices, int64_t* seeds, int64_t* seq_lens, const int64_t* loc,
                  int32_t* packed, int64_t* free_slots, int64_t* out, int64_t n_seeds, int bs, int K, int page,
                  const gss_finish_rule* finish, int32_t* cut, int32_t* n_free, gss_stream_t stream);

/* gss_kv_meta replaces _ss_kv_meta_kernel (patches/sglang/python/sglang/srt/speculative/selfspec_fast_attn.py:
 * 104-132): the flattened KV index list of a batch for page size 1.
 *   n_i           = seq_lens[i] + extra, clamped into [0, r2t_stride]
 *   kv_indptr     = [0, n_0, n_0 + n_1, ...]                                        int32 [bs + 1]
 *   kv_indices    = req_to_token[req_pool_indices[i], 0 .. n_i-1] at kv_indptr[i]    int32
 * req_to_token is int32 [n_req, r2t_stride]; rows whose pool index is outside [0, n_req) write no indices; entries
 * at or past kv_indices_cap are not written (the caller sizes the buffer from its host lengths, as the reference's
 * _meta does, selfspec_fast_attn.py:244-253).
 */
int gss_kv_meta(const int32_t* req_to_token, int64_t r2t_stride, int64_t n_req, const int64_t* req_pool_indices,
                const int64_t* seq_lens, int extra, int32_t* kv_indptr, int32_t* kv_indices,
                int64_t kv_indices_cap, int bs, gss_stream_t stream);

/* gss_log_append: the device-side round history of the graph-replayed decode loop (no counterpart in the
 * reference, which reads every round back to the host: src/fast_sampling.py:581-583). Row li = min(*ctr,
 * capacity - 1) of each log s (int32 [capacity, len_s]) receives src_s[0 .. len_s), then *ctr += 1. Up to three
 * logs; a NULL src skips its log. One launch of one workgroup. */
int gss_log_append(int64_t* ctr, int capacity, const int32_t* src0, int32_t* log0, int len0, const int32_t* src1,
                   int32_t* log1, int len1, const int32_t* src2, int32_t* log2, int len2, gss_stream_t stream);

/* ---------------------------------------------------------------- decoder-layer helpers -------------------------
 * Fused elementwise pieces of the GLM text decoder layer (transformers GlmOcrTextDecoderLayer, which the reference
 * calls through src/fast_sampling.py:89-102). bf16 in and out; fp32 inside; every step rounds to bf16 where the
 * reference's bf16 module does.
 *
 * gss_rope_stage: split the fused q|k|v projection rows, rotate q and k (interleaved pairs over the first rot_dim
 * dims, position = seq_lens[b] + (pos_delta ? pos_delta[b] : 0) + pos_offset + w), write q [bs, W, Hq, D] and the
 * window K/V [bs, W, Hkv, D].
 */
int gss_rope_stage(const void* qkv, int64_t ld_qkv, const int32_t* seq_lens, const int32_t* pos_delta,
                   int pos_offset, const float* inv_freq, int rot_dim, void* q, void* k_win, void* v_win, int bs,
                   int W, int Hq, int Hkv, int D, gss_stream_t stream);

/* gss_rope_stage_mrope: the same split and rotation for `rows` rows of one sequence with explicit M-RoPE positions
 * int32 [rows, 3] (t, h, w), as transformers GlmOcrTextRotaryEmbedding (modeling_glm_ocr.py:672-692): rotary
 * frequency i uses position component 0 when i < sec_t, 1 when i < sec_t + sec_h, else 2 (mrope_section). Used by
 * the prefill of image-token prompts, whose rows carry distinct (t, h, w) positions; the reference feeds them
 * through _run_layers (src/fast_sampling.py:499-503). Outputs q [rows, Hq, D], window K/V [rows, Hkv, D]. */
int gss_rope_stage_mrope(const void* qkv, int64_t ld_qkv, const int32_t* positions, int sec_t, int sec_h,
                         const float* inv_freq, int rot_dim, void* q, void* k_win, void* v_win, int rows, int Hq,
                         int Hkv, int D, gss_stream_t stream);

/* out = rmsnorm(x) * w  (GlmOcrRMSNorm), rows x H. */
int gss_rmsnorm(const void* x, const void* w, void* out, int rows, int H, float eps, gss_stream_t stream);

/* h[r] = table[ids[r]] (embed_tokens, src/fast_sampling.py:484), x[r] = rmsnorm(h[r]) * w: the embedding lookup of
 * a window and the first layer's input norm in one launch (bit-identical to the lookup followed by gss_rmsnorm).
 * table bf16 [V, H], ids int32 [rows]; an id outside [0, V) gives a zero row. */
int gss_embed_rmsnorm(const void* table, const int32_t* ids, int V, const void* w, void* h, void* x, int rows,
                      int H, float eps, gss_stream_t stream);

/* h = h + rmsnorm(a) * w_post;  x = rmsnorm(h) * w_next   (sandwich-norm residual, then the next norm). */
int gss_add_rmsnorm(const void* a, const void* w_post, void* h, const void* w_next, void* x, int rows, int H,
                    float eps, gss_stream_t stream);

/* gss_add_rmsnorm with a = bf16(parts[0] + ... + parts[n_parts - 1]) (fp32, added in part order; parts
 * [n_parts][rows][H], 16-byte aligned, as gss_gemm_parts writes them). H / 64 must be a multiple of 4;
 * 1 <= n_parts <= 4 (gss_gemm_parts writes at most 2), else GSS_ERR_UNSUPPORTED. */
int gss_add_rmsnorm_parts(const float* parts, int n_parts, const void* w_post, void* h, const void* w_next, void* x,
                          int rows, int H, float eps, gss_stream_t stream);

/* out[r, :F] = up * silu(gate) with gu[r] = [gate (F) | up (F)], row stride ld_gu elements (GlmOcrTextMLP). */
int gss_silu_mul(const void* gu, int64_t ld_gu, void* out, int rows, int F, gss_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GSS_H */
