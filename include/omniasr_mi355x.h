/*
 * omniasr_mi355x.h -- C ABI of the MI355X (gfx950) kernels of omniasr-trt's speculative greedy
 * decoder step.
 *
 * The reference's boundary is the Python module ``omniasr_trt.kernels``: functions taking torch
 * tensors and launching Triton kernels on torch's current stream. This library replaces those
 * kernels; each entry point below names the reference function (file:line, relative to the
 * reference repository) whose work it does. The Python shim ``omniasr-trt_amd/kernels.py`` keeps
 * the reference's function signatures and calls these entry points with raw device pointers.
 *
 * Conventions shared by every entry point:
 *   - pointers are device pointers; sizes, strides and positions are int64 (token buffers int32,
 *     flags uint8 holding 0/1 -- torch.bool's layout), strides count elements, not bytes;
 *   - ``stream`` is a hipStream_t (NULL: the default stream); nothing synchronises the host and
 *     nothing allocates, so every call can be captured into a HIP graph;
 *   - the return value is OMNI_OK, a negative OMNI_ERR_* for an argument the kernels do not cover
 *     (checked before anything is launched), or a positive hipError_t from the launch;
 *   - indices read from device memory (positions, cache rows, lengths) are clamped or skipped where
 *     they would leave a buffer, so a wrong index never makes a kernel touch memory outside the
 *     arguments' extents (the reference's behaviour there is undefined).
 */
#ifndef OMNIASR_MI355X_H
#define OMNIASR_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMNI_OK 0
#define OMNI_ERR_INVALID (-1)   /* null pointer, negative size, misaligned or too small stride */
#define OMNI_ERR_DTYPE (-2)     /* element type the kernels are not built for */
#define OMNI_ERR_SHAPE (-3)     /* head_dim / tokens / window beyond what the kernels cover */
#define OMNI_ERR_WORKSPACE (-4) /* workspace smaller than omni_verify_attention_workspace() */

#define OMNI_F32 0
#define OMNI_BF16 1

/* verify-attention flags */
#define OMNI_ATTN_SEPARATE_COMBINE 1 /* merge key splits in a second launch, not in the last split */
#define OMNI_ATTN_SPLIT_K 2          /* always split-K, never one workgroup per (head, row) */

/* Human-readable text of a status code (static storage). */
const char *omni_status_string(int status);

/* ABI version of this header (bumped on any signature change). */
int omni_abi_version(void);

/*
 * RoPE + KV-cache append.  Replaces ``kernels.rope_kv`` / ``_rope_kv``
 * (src/omniasr_trt/kernels.py:294-306, 31-54) with the rotation of ``apply_rope``
 * (src/omniasr_trt/modeling.py:301-306).
 *
 * Token n (0 <= n < n_tokens) of ``qkv`` [n_tokens, 3*heads*head_dim] (q | k | v, row stride
 * ``qkv_row_stride``) is rotated at position pos[n]: interleaved pairs (re, im) of q and k become
 * (re*c - im*s, re*s + im*c) in fp32 with c, s = cs[pos[n], j] (``cs`` [cs_rows, head_dim/2, 2]
 * fp32), each product rounded on its own (no fused multiply-add), then rounded to the element
 * type (bf16: nearest even).  The rotated q goes to ``q_out`` [n_tokens, heads, head_dim]; the
 * rotated k and the unrotated v go to cache row slots[n] (NULL: n), position cache_pos[n] (NULL:
 * pos[n]) of ``k_cache`` / ``v_cache`` (strides row / head / position, unit stride in head_dim).
 * head_dim: a multiple of 8.  dtype: OMNI_BF16 or OMNI_F32.
 */
int omni_rope_kv_append(const void *qkv, int64_t qkv_row_stride, const float *cs, int64_t cs_rows,
                        const int64_t *pos, const int64_t *slots, const int64_t *cache_pos,
                        void *q_out, void *k_cache, void *v_cache, int64_t stride_row,
                        int64_t stride_head, int64_t stride_pos, int64_t cache_rows,
                        int64_t cache_len, int64_t n_tokens, int32_t heads, int32_t head_dim,
                        int32_t dtype, void *stream);

/*
 * Key-split size (keys per split, a multiple of 32) that omni_verify_attention uses when called
 * with chunk = 0, for this launch shape.
 */
int32_t omni_verify_attention_chunk(int32_t rows, int32_t tokens, int32_t heads, int32_t head_dim,
                                    int32_t keys);

/* Bytes of workspace omni_verify_attention needs for this shape and split size (0: default). */
size_t omni_verify_attention_workspace(int32_t rows, int32_t tokens, int32_t heads,
                                       int32_t head_dim, int32_t keys, int32_t chunk);

/*
 * Multi-query split-K flash-decode verification attention.  Replaces ``kernels.draft_attention``
 * (``_beam_ctx`` with CAUSAL=True + ``_beam_combine``, src/omniasr_trt/kernels.py:338-358, 56-113,
 * 146-161) and, at tokens = 1, ``kernels.decode_attention`` (``_attn_split`` + ``_attn_combine``,
 * src/omniasr_trt/kernels.py:406-423, 163-211).
 *
 * ``q`` [rows*tokens, heads, head_dim] contiguous: row b's ``tokens`` queries are rows
 * b*tokens .. b*tokens+tokens-1.  Query i of row b attends to keys [0, lengths[b] + i) of cache
 * row b (``k_cache`` / ``v_cache`` with strides row / head / position, unit stride in head_dim,
 * ``cache_len`` positions): out = softmax(q.k * scale) . v, accumulated in fp32; an empty key range
 * gives zeros.  All keys must lie within the first ``keys`` positions (the graph bucket); the launch
 * grid depends on ``keys`` only.  One pass over a row's keys serves all of its queries.
 * ``chunk``: keys per split (a multiple of 32; 0: omni_verify_attention_chunk()); a row with n keys has
 * ceil(n / chunk) splits, and its 32-key tiles are dealt out round-robin over them.
 * ``workspace``: at least omni_verify_attention_workspace() bytes, 256-byte aligned, any content.
 * ``counters``: rows*heads int32, zero before the first call; every call leaves them zero (calls
 * that share them must not overlap in time).
 * Decomposition: with bf16, head_dim 128, contiguous key rows (stride_pos == head_dim), tokens <= 11,
 * rows <= 256 and rows * heads >= 128, one launch of rows*heads 8-wave workgroups: workgroup i takes the
 * first half of the i-th longest (head, row) and the second half of the i-th shortest, and the two halves
 * of each unit merge through the workspace and ``counters`` (``chunk`` unused; results do not depend on
 * timing).  With bf16, head_dim 256 or 512, contiguous key rows and rows <= 64: split-K with a fixed
 * budget of 256 workgroups (at least one per row) dealt to the rows of each head in proportion to their
 * key counts, the last split of each (row, head) merging the others through ``counters`` (``chunk`` and
 * OMNI_ATTN_SEPARATE_COMBINE unused; results do not depend on timing).  Otherwise, or when ``flags`` has
 * OMNI_ATTN_SPLIT_K, split-K as above.
 * bf16: head_dim 128, 256 or 512 with contiguous key rows runs on MFMA (256 / 512: a workgroup of one wave per
 * 128 dimensions, the partial scores added through LDS), any other multiple of 8 on the vector ALUs; f32:
 * vector ALUs (fp32 products).  tokens: 1..16 (1..32 for bf16 head dims 256 / 512 with contiguous key rows).
 */
int omni_verify_attention(const void *q, const void *k_cache, const void *v_cache,
                          int64_t stride_row, int64_t stride_head, int64_t stride_pos,
                          int64_t cache_len, const int64_t *lengths, int32_t rows, int32_t tokens,
                          int32_t heads, int32_t head_dim, int32_t keys, int32_t chunk, float scale,
                          void *out, void *workspace, size_t workspace_bytes, int32_t *counters,
                          int32_t flags, int32_t dtype, void *stream);

/* Capacity of the static scratch behind omni_verify_attention_static. */
#define OMNI_STATIC_WORKSPACE_BYTES ((size_t)32 << 20) /* split partials: 32 MiB per GPU */
#define OMNI_STATIC_MAX_UNITS 16384                    /* rows * heads (merge tickets) */

/*
 * omni_verify_attention without a caller's workspace or tickets: it allocates nothing (no hipMalloc, no
 * allocating library call), for callers that cannot allocate -- code under HIP graph capture that must not
 * call hipMalloc, tight serving loops, harnesses that forbid allocation.  No counterpart in the reference
 * (its Triton wrappers allocate their split workspace with torch.empty on every call, kernels.py:349-350).
 *
 * Arguments and results are those of omni_verify_attention with workspace, workspace_bytes and counters
 * taken away: the split partials and merge tickets live in a file-scope device array of the library
 * (OMNI_STATIC_WORKSPACE_BYTES of partials plus OMNI_STATIC_MAX_UNITS tickets), one copy per GPU, held
 * until the process ends.  A shape whose workspace (omni_verify_attention_workspace) exceeds
 * OMNI_STATIC_WORKSPACE_BYTES, or with rows * heads > OMNI_STATIC_MAX_UNITS, returns OMNI_ERR_WORKSPACE
 * before anything is launched.  Each call first clears the tickets with a fill kernel on ``stream``, then
 * launches what omni_verify_attention launches.  Every call on a GPU shares that GPU's array: calls that
 * overlap in time on one GPU (other streams, other threads) race and must not be made.  The array used is the
 * current device's (hipGetDevice), so ``stream`` must belong to the current device, as the caller's buffers do.
 * The array's device address is looked up once per device, by omni_verify_attention_static_init or else by the
 * first call on the device; a first call whose stream is being captured returns OMNI_ERR_INVALID without
 * launching anything (the lookup may load the code object, which a capture must not record).
 */
int omni_verify_attention_static(const void *q, const void *k_cache, const void *v_cache,
                                 int64_t stride_row, int64_t stride_head, int64_t stride_pos,
                                 int64_t cache_len, const int64_t *lengths, int32_t rows, int32_t tokens,
                                 int32_t heads, int32_t head_dim, int32_t keys, int32_t chunk, float scale,
                                 void *out, int32_t flags, int32_t dtype, void *stream);

/*
 * Set-up of omni_verify_attention_static on the current device: looks up the device address of its static array
 * (hipGetSymbolAddress) and keeps it.  Call it once per device, with that device current, before any graph
 * capture that records omni_verify_attention_static.  No counterpart in the reference; for the same callers
 * (those that cannot allocate).  Allocates nothing.
 */
int omni_verify_attention_static_init(void);

/* Bytes of workspace omni_beam_attention needs for this shape and split size (0: default). */
size_t omni_beam_attention_workspace(int32_t groups, int32_t beams, int32_t heads, int32_t head_dim,
                                     int32_t ctx_keys, int32_t chunk);

/*
 * Beam-search attention.  Replaces ``kernels.beam_attention`` (``_beam_ctx`` with CAUSAL=False,
 * ``_beam_gen``, ``_beam_combine``; src/omniasr_trt/kernels.py:309-332, 56-161) as called by
 * ``BeamDecoder.attention`` (src/omniasr_trt/beam.py:107-112).
 *
 * ``q`` [groups*beams, heads, head_dim] contiguous: group g's beams are rows g*beams .. g*beams+beams-1.
 * Row r = g*beams + i attends to the first ctx_len[g] keys of context row g (``k_ctx`` / ``v_ctx``,
 * strides ctx_row / ctx_head / ctx_pos, ``ctx_cap`` positions, all within ``ctx_keys``), and to its
 * generated keys j < gen_len[r], key j read at row ptr[r*ptr_stride + j] of ``k_gen`` / ``v_gen``
 * (strides gen_row / gen_head / gen_pos, ``gen_rows`` rows of ``gen_cap`` positions); pointers are
 * clamped into [0, gen_rows).  out = softmax(q.k * scale) . v over both parts, fp32 accumulation; no
 * key at all gives zeros.  One pass over a group's context serves all of its beams (the kernels of
 * omni_verify_attention with every query over the same keys).  bf16, head_dim 128, contiguous key rows,
 * beams <= 11 and groups * heads >= 128: the context halves kernel; bf16, head_dim 256 / 512, contiguous key rows,
 * groups <= 64: the balanced wide-head kernel (``counters``: groups*heads int32 tickets, zero before the first
 * call, left zero).  In both, when beams * gen_cap <= 4096 and the generated cache's byte offsets fit 32 bits,
 * each group's generated keys (beam 0's, then beam 1's, ...) are tiles of the same launch after its context;
 * otherwise they are read by a pointer-chasing launch into one more partial that the context's merge takes.
 * Other shapes: split-K and a merge launch.  ``chunk``: context keys per split (0: the library's choice).
 * ``workspace``: at least omni_beam_attention_workspace() bytes, 256-byte aligned.  beams: 1..16.
 */
int omni_beam_attention(const void *q, const void *k_ctx, const void *v_ctx, int64_t ctx_row,
                        int64_t ctx_head, int64_t ctx_pos, int64_t ctx_cap, const int64_t *ctx_len,
                        const void *k_gen, const void *v_gen, int64_t gen_row, int64_t gen_head,
                        int64_t gen_pos, int64_t gen_cap, int64_t gen_rows, const int32_t *ptr,
                        int64_t ptr_stride, const int64_t *gen_len, int32_t groups, int32_t beams,
                        int32_t heads, int32_t head_dim, int32_t ctx_keys, int32_t chunk, float scale,
                        void *out, void *workspace, size_t workspace_bytes, int32_t *counters,
                        int32_t dtype, void *stream);

/*
 * Each group's generated keys listed once per distinct (row, position).  No counterpart in the reference: the
 * beams of a group share most of their history (ptr rows copied from their parents, src/omniasr_trt/beam.py:
 * 170-187), so most generated keys are the same cache row and position for several beams; built once per search
 * step, the list lets omni_beam_attention_listed read each such key once for all the beams that see it.  For beam
 * decoders that call the attention layer by layer with one set of pointers per step.
 *
 * Group g (rows g*beams .. g*beams+beams-1; ``ptr``, ``gen_len``, ``gen_cap``, ``gen_rows`` as for
 * omni_beam_attention): list[g*list_stride + f] is the byte offset of key f from a generated cache's base, without
 * its head (row * gen_row + position * gen_pos elements, times 2), mask[g*list_stride + f] the beams that see it
 * (bit i: beam i), count[g] the list's length.  Order: by position, then by the first beam that reaches the key.
 * list_stride >= beams * gen_cap; beams: 1..16; the offsets must fit 32 bits (OMNI_ERR_SHAPE otherwise).
 */
int omni_beam_gen_list(int32_t groups, int32_t beams, const int32_t *ptr, int64_t ptr_stride, const int64_t *gen_len,
                       int64_t gen_cap, int64_t gen_rows, int64_t gen_row, int64_t gen_pos, uint32_t *list,
                       uint16_t *mask, int32_t *count, int64_t list_stride, void *stream);

/*
 * omni_beam_attention with the lists of omni_beam_gen_list (built from the same ptr / gen_len and the generated
 * caches' strides, on the same stream before the call): where the generated keys are tiles of the context launch,
 * they are each group's listed keys, each seen by the beams of its mask; elsewhere the lists are not used.  No
 * counterpart in the reference (see omni_beam_gen_list); the results equal omni_beam_attention's up to the order of
 * the floating-point sums.
 */
int omni_beam_attention_listed(const void *q, const void *k_ctx, const void *v_ctx, int64_t ctx_row,
                               int64_t ctx_head, int64_t ctx_pos, int64_t ctx_cap, const int64_t *ctx_len,
                               const void *k_gen, const void *v_gen, int64_t gen_row, int64_t gen_head,
                               int64_t gen_pos, int64_t gen_cap, int64_t gen_rows, const int32_t *ptr,
                               int64_t ptr_stride, const int64_t *gen_len, const uint32_t *gen_list,
                               const uint16_t *gen_mask, const int32_t *gen_count, int64_t list_stride,
                               int32_t groups, int32_t beams, int32_t heads, int32_t head_dim, int32_t ctx_keys,
                               int32_t chunk, float scale, void *out, void *workspace, size_t workspace_bytes,
                               int32_t *counters, int32_t dtype, void *stream);

/*
 * Causal attention over whole contexts: the prefill's
 *     F.scaled_dot_product_attention(q, k, v, is_causal=True)
 * (src/omniasr_trt/decode.py:163-164, after kernels.rope_kv has written the contexts' K / V into their cache
 * rows, decode.py:155-162).  Query p (0 <= p < width) of context b attends to keys [0, p] of cache row
 * slots[b] (clamped into [0, cache_rows)); q and out are [contexts * width, heads, head_dim] (context b's
 * queries at rows b*width .. b*width + width - 1, right padding computed like any other position).
 * K / V caches: element strides stride_row / stride_head / stride_pos, cache_len >= width positions.
 * bf16, head_dim 128, 256 or 512, contiguous key rows (stride_pos == head_dim); fp32 accumulation.  No workspace.
 * Head dim 128: one workgroup of 4 waves x 48 queries per 192-query block; 256 / 512: one workgroup of 8 waves per
 * 192 / 96-query block, each wave one 128-dimension slice, partial scores added through LDS and each 16-query
 * group's softmax run by one wave.
 */
int omni_prefill_attention(const void *q, const void *k_cache, const void *v_cache, int64_t stride_row,
                           int64_t stride_head, int64_t stride_pos, int64_t cache_len, int64_t cache_rows,
                           const int64_t *slots, int32_t contexts, int32_t width, int32_t heads,
                           int32_t head_dim, float scale, void *out, int32_t dtype, void *stream);

/*
 * Draft proposal of every row.  Replaces ``kernels.propose`` / ``_propose``
 * (src/omniasr_trt/kernels.py:361-377, 214-268) as called by ``SpecDecoder.propose``
 * (src/omniasr_trt/spec.py:76-80).
 *
 * Row b: the newest ``ngram`` tokens out[b, last[b] - t] (valid while >= first[b]) are matched
 * against ``anchor_width`` draft anchors (offset i - behind from next[b] - 1, live while the offset
 * is <= ahead and the anchor < draft_len[b]) and ``self_width`` earlier own positions
 * (last[b] - 1 - i, live while >= first[b]); a draft anchor needs reach[r][1] matching tokens
 * within distance reach[r][0] (r = 0..3, else ngram); the best anchor ranks score*256 - distance
 * (first on ties), the best own position is the latest with the most matches.  Writes prop[b, 0..k)
 * (int64), use_draft[b] and start[b] (draft position of the first proposal).
 * ``out`` [rows, out_stride] int32 (out_cap positions), ``draft`` [rows, draft_stride] int32
 * (draft_cap entries).  k <= 64, ngram <= 64, anchor_width and self_width <= 4096.
 */
int omni_propose(const int32_t *out, int64_t out_stride, int64_t out_cap, const int32_t *draft,
                 int64_t draft_stride, int64_t draft_cap, const int64_t *draft_len,
                 const int64_t *last, const int64_t *first, const int64_t *next, int64_t *prop,
                 uint8_t *use_draft, int64_t *start, int32_t rows, int32_t k, int32_t ngram,
                 int32_t behind, int32_t ahead, int32_t anchor_width, int32_t self_width,
                 int32_t self_min, const int32_t reach[8], void *stream);

/*
 * omni_propose plus the assembly of a drafted step's inputs, in the same launch.  Replaces
 * ``SpecDecoder.propose`` and the torch operations of ``SpecDecoder.step`` that build the fed
 * tokens, positions, cache rows and key counts (src/omniasr_trt/spec.py:85-95):
 *   running = !done[b]; p = last[b] + running;
 *   tokens[b] = (tok[b], prop[b, 0..k));             [rows, k+1] int64
 *   pos[b*(k+1) + j] = min(running ? p + j : last[b], capacity - 1);
 *   slots[b*(k+1) + j] = b;  lengths[b] = running ? p + 1 : 0.
 * ``prop`` may be NULL (the proposals then only land in ``tokens``).
 */
int omni_spec_prepare(const int32_t *out, int64_t out_stride, int64_t out_cap,
                      const int32_t *draft, int64_t draft_stride, int64_t draft_cap,
                      const int64_t *draft_len, const int64_t *last, const int64_t *first,
                      const int64_t *next, int64_t *prop, uint8_t *use_draft, int64_t *start,
                      int32_t rows, int32_t k, int32_t ngram, int32_t behind, int32_t ahead,
                      int32_t anchor_width, int32_t self_width, int32_t self_min,
                      const int32_t reach[8], const int64_t *tok, const uint8_t *done,
                      int64_t capacity, int64_t *tokens, int64_t *pos, int64_t *slots,
                      int64_t *lengths, void *stream);

/*
 * Greedy acceptance and rollback of a drafted step, from the argmaxes.  Replaces
 * ``kernels.accept`` / ``_accept`` (src/omniasr_trt/kernels.py:380-390, 271-291).
 *
 * Row b with done[b] == 0: p = last[b] + 1, g_j = nxt[b, j]; kept = the number of leading j with
 * tokens[b, j+1] == g_j (at most T-1); stop_j = (g_j == eos or p + j >= limit) and j <= kept;
 * n = the first j with stop_j, else kept.  Writes out[b, min(p + j, out_cap - 1)] = g_j for
 * j <= n, tok[b] = g_n, last[b] = p + n, done[b] = any stop_j and, when draft_next is not NULL,
 * draft_next[b] = (use_draft[b] ? start[b] : draft_next[b]) + n + 1.  Finished rows are untouched.
 * The cache is rolled back by the length alone: nothing is erased.  T: 1..64.
 */
int omni_accept(const int64_t *tokens, const int64_t *nxt, int32_t *out, int64_t out_stride,
                int64_t out_cap, int64_t *tok, int64_t *last, uint8_t *done, int64_t *draft_next,
                const int64_t *start, const uint8_t *use_draft, int32_t rows, int32_t tokens_per_row,
                int64_t limit, int64_t eos, void *stream);

/*
 * Verify logits -> greedy argmax -> acceptance.  Replaces
 * ``F.log_softmax(logits, -1).argmax(-1)`` of the drafted step (src/omniasr_trt/spec.py:106-107)
 * and of the one-token step (src/omniasr_trt/decode.py:218-224), followed by omni_accept.
 *
 * ``logits`` [rows*T, vocab] (row stride ``logits_stride``, element type ``logits_dtype``): the
 * argmax of row r is the first index i where the log-softmax, computed as PyTorch's does
 * ((x_i - max) - log(sum_j exp(x_j - max)) in fp32, then rounded to the logits' type), reaches its
 * maximum.  It is written to nxt[r] (int64) when ``nxt`` is not NULL, then every row is accepted as
 * by omni_accept.  ``start``, ``use_draft`` and ``draft_next`` may be NULL together (the one-token
 * step).  T: 1..64.  With ``nxt`` and a vocabulary up to 32768 bf16 / 16384 fp32 entries, two
 * launches (an argmax workgroup per row, then the acceptance); otherwise one (a workgroup per slot),
 * for vocabularies up to 131072 bf16 / 65536 fp32 entries.
 */
int omni_greedy_accept(const void *logits, int64_t logits_stride, int32_t vocab,
                       int32_t logits_dtype, const int64_t *tokens, int64_t *nxt, int32_t *out,
                       int64_t out_stride, int64_t out_cap, int64_t *tok, int64_t *last,
                       uint8_t *done, int64_t *draft_next, const int64_t *start,
                       const uint8_t *use_draft, int32_t rows, int32_t tokens_per_row,
                       int64_t limit, int64_t eos, void *stream);

/*
 * The beam step's bookkeeping before its layers.  Replaces the torch ops of ``BeamDecoder.step_beam``
 * before the layers (src/omniasr_trt/beam.py:127-145: live rows, positions, key counts, the row's own
 * pointer at the position it writes).
 *
 * Rows r = g*beams + i of groups g < groups: live = !group_done[g], k = k_step[g];
 * pos[r] = ctx[g] + k - 1, gen_pos[r] = max(k - 1, 0), gen_len[r] = live ? k : 0,
 * ctx_len[g] = group_done[g] ? 0 : ctx[g], and for live rows ptr[r*ptr_stride + gen_pos[r]] = r (rows whose
 * gen_pos is not below ptr_cols are left alone).  beams: 1..16.
 */
int omni_beam_prepare(int32_t groups, int32_t beams, const int64_t *ctx, const int64_t *k_step,
                      const uint8_t *group_done, int32_t *ptr, int64_t ptr_stride, int64_t ptr_cols,
                      int64_t *pos, int64_t *gen_pos, int64_t *ctx_len, int64_t *gen_len, void *stream);

/*
 * The beam step's bookkeeping after the per-group top-``beams`` of the offers.  Replaces the torch ops
 * of ``BeamDecoder.step_beam`` after the top-k and the parent reorder (src/omniasr_trt/beam.py:159-187).
 *
 * ``best`` / ``flat``: torch.topk(offers.view(groups, beams * vocab), beams) values (fp32 or fp64, as the
 * row scores: ``score_bytes`` 4 or 8) and indices.  Row r = g*beams + i, live = !group_done[g],
 * k = k_step[g]: parent = live ? g*beams + flat[r] / vocab : r, chosen = live ? flat[r] % vocab : tok[r],
 * EOS when ended[parent]; row r's ptr and hist rows (``ptr_cols`` / ``hist_cols`` columns) become the
 * parent's, and a live row's hist[r][k] = chosen; extends = live && !ended[parent]: score[r] = extends ?
 * best[r] : score[parent], count[r] = count[parent] + (extends && chosen != pad && chosen != eos),
 * ended[r] = live ? chosen == eos : ended[parent], tok[r] = chosen.  Then k_step[g] += live and
 * group_done[g] |= all rows of g ended || ctx[g] + k_step[g] - 2 >= limit.  Values are moved, never
 * recomputed, so the state equals the torch ops' bit for bit.  beams: 1..16.
 */
int omni_beam_take_over(int32_t groups, int32_t beams, int64_t vocab, const void *best, const int64_t *flat,
                        int32_t *ptr, int64_t ptr_stride, int64_t ptr_cols, int32_t *hist,
                        int64_t hist_stride, int64_t hist_cols, uint8_t *ended, void *score,
                        int32_t score_bytes, int64_t *count, int64_t *tok, int64_t *k_step,
                        uint8_t *group_done, const int64_t *ctx, int64_t limit, int32_t eos, int32_t pad,
                        void *stream);

/* Bytes of workspace omni_beam_select needs: groups x beams x beams pairs of 8 bytes. */
size_t omni_beam_select_workspace(int32_t groups, int32_t beams);

/* What omni_beam_select's input rows hold. */
#define OMNI_SELECT_LOGP 0   /* log-probabilities (the caller's F.log_softmax): the choice is the reference's exactly */
#define OMNI_SELECT_LOGITS 1 /* logits: the log-softmax runs in the kernel, in its own summation order */

/*
 * The beam step's choice (src/omniasr_trt/beam.py:165-175, after the LM head): for each of ``groups`` groups of
 * ``beams`` rows of ``logits`` [groups * beams, vocab] (bf16, row stride ``logits_stride``), logp = the rows
 * themselves (``input_kind`` OMNI_SELECT_LOGP: the output of the reference's own F.log_softmax, beam.py:162) or the
 * log_softmax of each row computed here (OMNI_SELECT_LOGITS: fp32 max and sum of exp in this kernel's order,
 * logsum = log(sum), logp = bf16((x - max) - logsum); a logp on a bf16 rounding boundary can round differently from
 * torch's); the offers score + logp, or with ``length_norm`` once the group's row 0 has count > 0,
 * (score * count + logp) / (count + 1), each operation rounded to fp32 in that order; a row with ``ended`` set
 * offers only EOS (``eos``), at its score; then best [groups, beams] fp32 and flat [groups, beams] int64 =
 * offers.view(groups, beams * vocab).topk(beams), best first, equal values in the order of their flat index.
 * Replaces the offers' torch ops and torch.topk (and, with OMNI_SELECT_LOGITS, F.log_softmax); the bookkeeping that
 * follows is omni_beam_take_over.  score fp32 [rows], count int64 [rows], ended uint8 [rows].  ``workspace``:
 * omni_beam_select_workspace() bytes; ``tickets``: one int per group, zero, left zero (calls that overlap on one
 * GPU need tickets of their own).  beams 1..16; vocab a multiple of 8, at most 16384; dtype OMNI_BF16.
 */
int omni_beam_select(const void *logits, int64_t logits_stride, int32_t groups, int32_t beams, int32_t vocab,
                     const float *score, const int64_t *count, const uint8_t *ended, int32_t length_norm,
                     int64_t eos, float *best, int64_t *flat, void *workspace, size_t workspace_bytes,
                     int32_t *tickets, int32_t input_kind, int32_t dtype, void *stream);

/*
 * RMS norm of each row: y[r][i] = x[r][i] * rsqrt(sum_j x[r][j]^2 / dim + eps) * weight[i], fp32 arithmetic,
 * one rounding to bf16 after both products.  Replaces the torch kernel of the decoder layers' RMSNorm
 * (``F.rms_norm``; the RMSNorm of src/omniasr_trt/modeling.py, run by SpecDecoder.step,
 * src/omniasr_trt/spec.py:97-106), which the reference leaves to torch; no counterpart among its kernels.
 * dim: a multiple of 8, at most 8192; strides in elements, multiples of 8.  dtype: OMNI_BF16.
 */
int omni_rms_norm(const void *x, int64_t x_stride, const void *weight, void *y, int64_t y_stride,
                  int32_t rows, int32_t dim, float eps, int32_t dtype, void *stream);

/*
 * The gated FFN's activation: out[r][i] = inner * bf16(silu(gate)), gate = gate_inner[r][i],
 * inner = gate_inner[r][ffn + i] (the fused gate|inner projection's halves, src/omniasr_trt/decode.py:34-54),
 * silu(g) = g / (1 + exp(-g)) in fp32 rounded to bf16, then the product in fp32 rounded to bf16 -- the
 * rounding of torch's ``inner * F.silu(gate)`` (src/omniasr_trt/spec.py:97-106), which the reference leaves
 * to torch; no counterpart among its kernels.  ffn: a multiple of 8; strides multiples of 8.  dtype: OMNI_BF16.
 */
int omni_silu_mul(const void *gate_inner, int64_t gate_inner_stride, void *out, int64_t out_stride,
                  int32_t rows, int32_t ffn, int32_t dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNIASR_MI355X_H */
