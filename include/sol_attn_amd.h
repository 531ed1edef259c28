/* C-ABI of the MI355X-native SOL routed-attention library (libsol_attn_amd.so).
 *
 * The reference binds its device work through a Python launch layer
 * (src/sol_attn_amd/kernels.py:185-225: `_pooled`, `launch_dense`,
 * `launch_sol`).  These entry points replace that layer one for one; the
 * public Python API above them (attention.py, indexed.py) is unchanged.
 *
 * Conventions
 *  - Tensors are BF16 (passed as `const void*`), FP32 (`float*`), int32,
 *    uint8 (bool) or int64, all in device memory of the current HIP device.
 *  - Q/K/V are addressed as rows of `head_dim` contiguous elements.  Each
 *    operand takes three element strides {batch, token, head}.  When an index
 *    pointer ([batch, tokens] int64, device memory) is given, token t of
 *    batch b is row index[b * tokens + t] and the batch stride is ignored
 *    (indexed windows, indexed.py:99).  sequence_length is then the number
 *    of rows the index may address: the caller validates its indices (as
 *    IndexedPlan.create does), and an entry outside [0, sequence_length) --
 *    a plan changed after validation -- is clamped into that range, so every
 *    access stays inside the caller's tensors.
 *  - Ragged indexed windows: key_lengths (int32 [batch], device memory; NULL =
 *    every entry has key_tokens keys) gives entry b's key count, 1..key_tokens;
 *    its keys are the first key_lengths[b] rows of its key_index row, and every
 *    buffer keeps the key_tokens-sized layout (out-of-range values are clamped
 *    into 1..key_tokens).  The reference supports equal-length windows only;
 *    this runs windows of different key counts in one call.
 *  - Row starts must be 16-byte aligned: base pointers 16-byte aligned and
 *    strides multiples of 8 elements.
 *  - The library never allocates or frees device memory.  Launches are
 *    asynchronous on `stream` (a hipStream_t; NULL = legacy default stream).
 *  - Return value: 0 on success, negative for an invalid argument (message in
 *    sol_last_error()), positive = the hipError_t of a failed launch.
 *  - Calls are stateless and re-entrant; results are deterministic (no
 *    floating-point atomics; fixed reduction orders).
 */
#ifndef SOL_ATTN_AMD_H
#define SOL_ATTN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SOL_ABI_VERSION 14
#define SOL_BLOCK 64                /* tokens per physical block, kernels.py:12 */
#define SOL_MAX_KEY_TOKENS (1ll << 25) /* key_tokens of one pooling call (2^19 key blocks) */

#define SOL_NOALLOC_SCRATCH_BYTES (128ll << 20) /* device workspace of sol_attention_noalloc */

#define SOL_OK 0
#define SOL_ERR_INVALID (-1)
#define SOL_ERR_UNSUPPORTED (-2)

/* ABI version of the loaded library (SOL_ABI_VERSION). */
int sol_abi_version(void);

/* Message of the last failure on the calling thread ("" if none). */
const char* sol_last_error(void);

/* Byte sizes of the pooling outputs for a problem (reference: the torch.empty
 * calls of kernels.py:187,207,211-212), with NKB = ceil(key_tokens / 64) key
 * blocks and NCT = ceil(NKB / 64) centroid tiles:
 *   sizes[0] ctiles      bf16 [batch, heads, NCT, 2, 64 * head_dim]  block centroids
 *   sizes[1] tiles       bf16 [batch, heads, NKB, 2, 64 * head_dim]  K and V block tiles
 *   sizes[2] chunk_sums  fp32 [batch, heads, ceil(NKB/16), 2, head_dim]
 *   sizes[3] key_mean    fp32 [batch, heads, head_dim]  (key_var has the same size)
 * Tile pairs: a K tile then a V tile, 64 rows x head_dim each, in 16-byte
 * chunks (8 features): K chunk c of row r at chunk c ^ (r & 15) (head_dim 128)
 * or c ^ ((r >> 1) & 7) (head_dim 64) of the row; V chunk c of row r at chunk
 * (r >> 2) * head_dim / 2 + (c >> 2) * 16 + (r & 3) * 4 + (c & 3) of the tile
 * (row quads).  Rows past the last key / block are zero.
 * The block tiles are needed only when the attention kernels cannot read
 * key blocks straight from K and V ("rows mode", see sol_attention_fwd):
 * indexed or ragged keys, fewer than 64 keys, token strides of 2^24 elements
 * or more. */
int sol_pool_sizes(int64_t batch, int64_t key_tokens, int64_t heads, int64_t head_dim,
                   int64_t sizes[4]);

/* K/V block pooling, attention tiles and diagonal key moments, in one pass over
 * K and V.  Replaces `_pooled(k)`, `_pooled(v)` (kernels.py:185-190, kernel
 * `_pool` kernels.py:16-27) and `_moments` (kernels.py:30-49).
 * sequence_length: rows key_index may address (ignored without key_index).
 * ctiles receives the BF16 (round-to-nearest-even) 64-token block means of K
 * and V (NULL: tiles only); tiles (NULL: none) receives every key block as the
 * tile pair the attention kernels stream in tiles mode; when
 * key_mean/key_var/chunk_sums are all non-NULL, also the per-(batch, head,
 * feature) population mean and clamped variance of the BF16 key centroids. */
int sol_pool_kv(const void* k, const int64_t* k_strides,
                const void* v, const int64_t* v_strides,
                const int64_t* key_index, const int32_t* key_lengths,
                int64_t sequence_length, int64_t batch, int64_t key_tokens,
                int64_t heads, int64_t head_dim, void* ctiles, void* tiles,
                float* chunk_sums, float* key_mean, float* key_var,
                void* stream);

/* Workspace bytes of sol_pair_strides (0: pairing does not apply, i.e. fewer
 * than 4 or more than 8192 query blocks, or an unsupported shape).
 * No counterpart in the reference (see sol_pair_strides). */
int64_t sol_pair_workspace_size(int64_t batch, int64_t query_tokens, int64_t heads,
                                int64_t head_dim);

/* Query-block pairing for sol_attention_fwd.  Its workgroups hold two query
 * blocks each and stream the union of their selected key blocks, so pairing
 * blocks with similar selections shortens the stream.  Per (batch entry,
 * head) this picks the stride s in 1..256 at which sol_attention_fwd pairs
 * query blocks (block i with block i + s inside each run of 2 s blocks,
 * adjacent pairs after the last full run): the one whose pairs have the most
 * alike normalised query-block means (routing follows those means).  s = 1
 * is the adjacent pairing.  Q and query_index as in sol_attention_fwd;
 * workspace: sol_pair_workspace_size() bytes, 16-byte aligned; strides:
 * int32 [batch, heads].  query_means: NULL, or fp32 [batch, heads,
 * ceil(query_tokens / 64), head_dim] receiving the FP32 query-block means
 * (torch's cascade summation order: bit-identical to the reference oracle's
 * `_means`, reference.py:13-15), which sol_attention_fwd's routing kernel
 * can take instead of reading Q again.  The pairing never changes results,
 * only the schedule.  No counterpart in the reference (one Triton program
 * per query block, no pairing). */
int sol_pair_strides(const void* q, const int64_t* q_strides, const int64_t* query_index,
                     int64_t sequence_length, int64_t batch, int64_t query_tokens,
                     int64_t heads, int64_t head_dim, void* workspace, int32_t* strides,
                     float* query_means, void* stream);

/* Workspace bytes of sol_key_covariance (0: unsupported shape). */
int64_t sol_key_covariance_workspace_size(int64_t batch, int64_t heads, int64_t head_dim);

/* Full population covariance of the BF16 key centroids per (batch entry,
 * head): cov = mean_j Kc_j Kc_j^T - mu mu^T, fp32 [batch, heads, head_dim,
 * head_dim], from the centroid tiles and key_mean of sol_pool_kv (moments
 * on); key_lengths as in sol_pool_kv.  For the full-covariance threshold
 * experiment of the reference's roadmap (ROADMAP.md:14-16), which the
 * reference does not implement; its diagonal is the `_moments` variance
 * (kernels.py:30-49) before clamping. */
int sol_key_covariance(const void* ctiles, const float* key_mean, const int32_t* key_lengths,
                       int64_t batch, int64_t key_tokens, int64_t heads, int64_t head_dim,
                       void* workspace, float* key_cov, void* stream);

/* Bytes of the split_workspace sol_attention_fwd takes for a problem (0:
 * the problem is not split, pass NULL).  Launches with at least two
 * query-sink blocks and at most a quarter of the query blocks, at most
 * 524,288 keys, and either fewer than 512 query-block pairs over all (entry,
 * head) pairs (finite beta) or beta = +INFINITY and at most 8,192 query
 * blocks, split the key blocks of sink blocks [0, 2 floor(sink blocks / 2))
 * over up to 8 workgroups each (parts of at least 16 blocks); a merge kernel
 * combines their partial softmax states.  Split launches pair adjacent query
 * blocks (pair_strides is ignored).
 * A sink block selects every key block, so without the split its workgroup
 * ends long after the rest of a short launch.  The size is an upper bound
 * for every workgroup_form.  Launches the small-launch kernel takes (see
 * sol_attention_fwd's workgroup_form) split inside their workgroups and
 * return 0.  No counterpart in the reference (one Triton program per query
 * block). */
int64_t sol_split_workspace_size(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                                 int64_t head_dim, double beta, int64_t query_sink_tokens);

/* Bytes of the route_workspace sol_attention_fwd may take (0 for beta =
 * -INFINITY, which selects every block, or an invalid shape): the routing
 * decisions, uint32 [batch, heads, ceil(query_tokens / 64), ceil(NKB / 32)]
 * (bit j of word w: key block 32 w + j), written by the routing kernel and
 * read by the attention kernel of the same call; then, 256-byte aligned,
 * int32 [batch, heads, ceil(query_tokens / 64)]: the order in which a
 * two-block launch hands its query tiles to the XCDs, formed from the
 * decisions (costly tiles first, each XCD's share of every head balanced;
 * the results do not depend on it). */
int64_t sol_route_workspace_size(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                                 double beta);

/* Routing + attention over the pooled keys of sol_pool_kv.  With a
 * route_workspace, a routing kernel forms the cutoffs and every (query block,
 * key block) decision first and the attention kernel reads them; without
 * one, the attention kernel routes each centroid tile as it streams it.
 * Decisions agree to the routing band (FP32 summation order), outputs are
 * otherwise the same.
 * Replaces the `_threshold` and `_sol` launches of `launch_sol`
 * (kernels.py:203-225; kernels kernels.py:52-64 and 101-182).
 * beta: finite, -INFINITY (every block exact) or +INFINITY (protected blocks
 * only); key_mean/key_var are read only for finite beta.  key_cov: NULL (the
 * reference's diagonal estimator, sqrt(sum Qc^2 var)) or fp32 [batch, heads,
 * head_dim, head_dim] from sol_key_covariance (the full-covariance threshold
 * experiment, sqrt(max(Qc^T cov Qc, 0))).  local_blocks < 0
 * disables the local band (indexed windows).  Sink token counts round
 * outward to whole blocks.  protection: NULL or uint8 [batch, NQB, NKB].
 * pair_strides: NULL (adjacent query blocks share a workgroup) or int32
 * [batch, heads] from sol_pair_strides (any value is a valid pairing).
 * split_workspace: NULL (no split) or 16-byte aligned device memory of
 * sol_split_workspace_size(batch, query_tokens, key_tokens, heads, head_dim,
 * beta, query_sink_tokens) bytes when that is nonzero; split and unsplit
 * calls agree to rounding (the parts' states merge in a fixed order).
 * route_workspace: NULL (routing inside the attention kernel, the better
 * choice for short launches) or 16-byte aligned device memory of
 * sol_route_workspace_size(batch, query_tokens, key_tokens, heads, beta)
 * bytes (routing kernel first: it saves the attention kernel a routing pass
 * and a barrier per centroid tile on long key sequences).  query_means: NULL
 * (the routing kernel forms the query-block means from Q) or the query_means
 * output of sol_pair_strides for the same Q (only with route_workspace).
 * out: contiguous BF16 [batch, query_tokens, heads, head_dim]; or, when
 * out_index (int64 [batch, query_tokens], device) is given, a contiguous BF16
 * [N, heads, head_dim] whose row out_index[b * query_tokens + t] receives
 * query t of entry b (the scatter `out[rows] = result` of a window adapter,
 * integrations/vdn.py:67-74, fused into the store; rows must be distinct;
 * rows outside [0, sequence_length) are not stored).  sequence_length: the
 * rows query_index may address and out_index's N (ignored without either).
 * counts: NULL or int32 [batch, NQB, heads] exact-block counts.
 * debug_selected (uint8) / debug_proxy (fp32): NULL or [batch, NQB, heads, NKB]
 * routing decisions and proxies (natural-log units); debug_cutoff: NULL or
 * fp32 [batch, NQB, heads].  Debug outputs are for verification, not timing.
 * qk_int8_tiles / qk_int8_scales: NULL (BF16 scores, the reference's
 * arithmetic) or the output of sol_quantize_keys: the quantised-QK
 * experiment of the reference's roadmap (ROADMAP.md:14-16; not implemented by
 * the reference), where exact blocks take S = s_q s_k (Q8 . K8) on the INT8
 * matrix cores, Q8 = the query row at one scale s_q = max|q| / 127; routing,
 * centroid terms and P V stay BF16; sol_quantize_keys's rows_mode must be
 * nonzero exactly when tiles is NULL here.
 * workgroup_form: 0 picks the schedule by launch size: launches at finite
 * or +INFINITY beta of at most 256 query blocks (over all entries and
 * heads) whose keys span at most
 * 64 (head_dim 64) or 32 (head_dim 128) blocks run one query block per
 * workgroup with its key tiles split over 4 (2) groups of two waves, merged
 * in LDS (outputs agree with the other forms to rounding; decisions and
 * counts are the same); otherwise one query block per workgroup below 512
 * query-block pairs, else 2.  1 or 2 force one or two query blocks per
 * workgroup without the key split (bit-identical results).  No counterpart
 * in the reference (one Triton program per query block).
 * ctiles / key_mean / key_var: NULL at beta = -INFINITY (unused), or where
 * sol_attention_pools_keys holds for the sizes and the call has plain K / V
 * rows (tiles, key_lengths, query_index, key_cov, INT8 tiles and
 * route_workspace NULL; workgroup_form 0): the attention launch then forms
 * the block centroids and diagonal moments itself, bit for bit as
 * sol_pool_kv does, and the whole call is one kernel launch.
 * Key blocks: with tiles NULL ("rows mode") the kernels DMA each key block's
 * rows straight from k / v (strides {batch, token, head} as in sol_pool_kv;
 * requires key_index-free, equal-length keys: key_lengths NULL, key_tokens >=
 * 64, token strides below 2^24 elements); otherwise from the tile pairs
 * sol_pool_kv wrote, and k / v are ignored (may be NULL). */
/* 1 when sol_attention_fwd over plain K / V rows of these sizes pools the
 * keys inside its one attention launch (ctiles, key_mean and key_var may be
 * NULL): head_dim 64, at least 64 and at most 1,024 keys (one pooling chunk
 * of 16 blocks) in a launch of the small-launch kernel (workgroup_form).  0
 * otherwise.  No counterpart in the reference: it launches `_pool`,
 * `_moments`, `_threshold` and `_sol` separately (kernels.py:203-225). */
int sol_attention_pools_keys(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                             int64_t head_dim);

int sol_attention_fwd(const void* q, const int64_t* q_strides, const int64_t* query_index,
                      int64_t sequence_length, int64_t batch, int64_t query_tokens, int64_t key_tokens,
                      const int32_t* key_lengths, int64_t heads, int64_t head_dim,
                      const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      const void* tiles, const void* ctiles,
                      const float* key_mean, const float* key_var, const float* key_cov,
                      const uint8_t* protection, const int32_t* pair_strides, void* split_workspace,
                      void* route_workspace, const float* query_means, double scale, double beta,
                      int64_t local_blocks,
                      int64_t kv_sink_tokens, int64_t query_sink_tokens,
                      void* out, const int64_t* out_index, int32_t* counts,
                      uint8_t* debug_selected, float* debug_proxy, float* debug_cutoff,
                      const void* qk_int8_tiles, const float* qk_int8_scales,
                      int workgroup_form, void* stream);

/* INT8 K tiles for the quantised-QK experiment of sol_attention_fwd: per key
 * block of K (k, k_strides, key_index, key_lengths, sequence_length as in
 * sol_pool_kv), one scale s_k = max|K| / 127 over the block's keys
 * (k8_scales, fp32 [batch, heads, NKB]) and K8 = rint(K * 127 / max|K|)
 * clamped to +-127 (k8_tiles, int8 [batch, heads, NKB, 64 * head_dim];
 * 16-byte chunk c of row r at chunk c ^ ((r >> 1) & 7) for head_dim 128,
 * c ^ ((r >> 2) & 3) for 64).  Row r of block j's tile is key 64 j + r (zero
 * past the end), except with rows_mode (for a rows-mode sol_attention_fwd
 * call, whose partial last block holds the sequence's last 64 keys): there
 * the partial last block's tile holds keys key_tokens - 64 + r, quantised
 * with the block's own scale.  No counterpart in the reference
 * (ROADMAP.md:14-16 asks for the experiment). */
int sol_quantize_keys(const void* k, const int64_t* k_strides, const int64_t* key_index,
                      const int32_t* key_lengths, int64_t sequence_length, int64_t batch,
                      int64_t key_tokens, int64_t heads, int64_t head_dim, int rows_mode,
                      void* k8_tiles, float* k8_scales, void* stream);

/* Packed-block protection of indexed windows, built on the GPU: the
 * protection part of `IndexedPlan.create` (indexed.py:27-62).  Block (w, qb,
 * kb) of protected_blocks (uint8 [windows, NQB, NKB]) is 1 when one of the
 * window's keys at positions 64 kb .. 64 kb + 63 (and below its key count)
 * has an original index inside [rows[w, 64 qb] - local_tokens,
 * rows[w, last row of qb] + local_tokens] or inside a protected range.
 * rows: int64 [windows, query_rows]; keys: int64 [windows, key_count]; both
 * strictly increasing per window (over a window's first key_lengths[w] keys
 * when key_lengths, int32 [windows], is given; later positions are never
 * read).  ranges: int64 [nranges, 2] ranges [a, b), NULL when nranges is 0.
 * All pointers are device memory.  Indices are not validated here: the
 * Python layer checks them first, as `IndexedPlan.create` does. */
int sol_plan_protection(const int64_t* rows, const int64_t* keys, const int32_t* key_lengths,
                        int64_t windows, int64_t query_rows, int64_t key_count,
                        int64_t local_tokens, const int64_t* ranges, int64_t nranges,
                        uint8_t* protected_blocks, void* stream);

/* Non-causal BF16 attention over all keys, FP32 softmax and accumulation.
 * Replaces `launch_dense` (kernels.py:193-200; kernel kernels.py:67-98).
 * tiles: NULL when the keys qualify for rows mode (key_tokens >= 64, token
 * strides below 2^24 elements; see sol_attention_fwd), else a workspace of
 * sol_pool_sizes()[1] bytes (filled here).
 * query_index: NULL, or int64 [batch, query_tokens] token rows of a
 * [sequence_length, heads, head_dim] Q (its token and head strides; the batch
 * stride is ignored), clamped into the sequence -- the gathered queries of
 * `out[rows] = dense(q[rows], k, v)` (integrations/vdn.py:57-61, the
 * anchor-row and global queries of a window adapter).
 * out: contiguous BF16 [batch, query_tokens, heads, head_dim], or with
 * out_index (int64 [batch, query_tokens]) a contiguous BF16
 * [sequence_length, heads, head_dim] whose row out_index[b, t] receives query
 * (b, t); entries outside [0, sequence_length) are not stored.  Keys are the
 * K / V rows as given (one contiguous token range per call: pass that
 * range's first row). */
int sol_dense_fwd(const void* q, const int64_t* q_strides,
                  const int64_t* query_index, int64_t sequence_length,
                  const void* k, const int64_t* k_strides,
                  const void* v, const int64_t* v_strides,
                  int64_t batch, int64_t query_tokens, int64_t key_tokens,
                  int64_t heads, int64_t head_dim, double scale,
                  void* tiles, void* out, const int64_t* out_index, void* stream);

/* Bytes of caller workspace sol_attention_all_in needs for these sizes: 0
 * when the attention launch pools its keys itself (sol_attention_pools_keys),
 * otherwise the sol_pool_kv buffers it uses, each 256-byte aligned (the
 * centroid tiles; the block tiles outside rows mode, which k_token_stride /
 * v_token_stride -- K's and V's token strides in elements -- and key_tokens
 * decide as in sol_attention_fwd; chunk sums and moments at finite beta) and
 * the split workspace (sol_split_workspace_size).  -1 for invalid sizes.
 * No counterpart in the reference. */
int64_t sol_attention_workspace_size(int64_t batch, int64_t query_tokens, int64_t key_tokens,
                                     int64_t heads, int64_t head_dim, double beta,
                                     int64_t query_sink_tokens, int64_t k_token_stride,
                                     int64_t v_token_stride);

/* All-in SOL attention in one call: sol_pool_kv followed by
 * sol_attention_fwd over BTHD inputs (no index, plan protection, covariance,
 * INT8 tiles or debug outputs; routing inside the attention kernel; one
 * launch when sol_attention_pools_keys holds), with the pooled key buffers
 * carved from `workspace` (sol_attention_workspace_size bytes, 16-byte
 * aligned; NULL when that size is 0).  Replaces the two calls of the launch
 * layer's `_sol` path (src/sol_attn_amd/kernels.py:203-225: pooling, moments,
 * threshold and `_sol`) for launches that need no query-block pairing: it
 * saves the host one call and its argument packing, which short launches
 * (tens of microseconds of GPU work) feel.  Results are bit-identical to
 * sol_pool_kv + sol_attention_fwd with the same workspace layout.  out:
 * contiguous BF16 [batch, query_tokens, heads, head_dim]; counts: NULL or
 * int32 [batch, NQB, heads]; other arguments as in sol_attention_fwd. */
int sol_attention_all_in(const void* q, const int64_t* q_strides,
                         const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides,
                         int64_t batch, int64_t query_tokens, int64_t key_tokens,
                         int64_t heads, int64_t head_dim, double scale, double beta,
                         int64_t local_blocks, int64_t kv_sink_tokens,
                         int64_t query_sink_tokens, void* workspace, int64_t workspace_bytes,
                         void* out, int32_t* counts, void* stream);

/* All-in SOL attention that allocates nothing: sol_pool_kv followed by
 * sol_attention_fwd (BTHD inputs; no index, plan protection, covariance or
 * debug outputs), with the pooled key buffers in a library-owned device array
 * of SOL_NOALLOC_SCRATCH_BYTES per GPU instead of caller workspace.  Same
 * results as those two calls (bit-identical).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  The caller passes Q/K/V, out (contiguous BF16 [batch,
 * query_tokens, heads, head_dim]) and counts (NULL or int32 [batch, NQB,
 * heads]); arguments as in sol_attention_fwd.  The pooled keys are the
 * centroid tiles, head_dim / 16 bytes per key token and head (padded to
 * whole 64-block tiles), and the moments; key blocks are read straight from K
 * and V (rows mode), except for fewer than 64 keys or token strides of 2^24
 * elements or more, where the block tiles (4 * head_dim bytes per key token
 * and head) join them, and the split workspace when the problem is split
 * (sol_split_workspace_size); routing runs inside the attention kernel.
 * Problems needing more than SOL_NOALLOC_SCRATCH_BYTES (128 MiB), and
 * arguments sol_attention_fwd would reject, return an error before any GPU
 * work.  Every call on one GPU shares that GPU's array: calls that overlap on
 * one GPU (different streams or threads) race and must be serialised by the
 * caller.  The array belongs to the library's device code object: it holds
 * 128 MiB on every GPU where the library's kernels are loaded (from the first
 * call on that GPU until the process ends), whether or not this entry point
 * is ever called.  Some attention kernel
 * variants (head_dim 128) keep a few values in per-lane private memory
 * (register spills); the HIP runtime provides that memory per queue and may
 * size it at the first launch of such a kernel on a queue, which is the
 * runtime's allocation, not this library's -- a caller that must not see
 * one makes any SOL call on the queue beforehand. */
int sol_attention_noalloc(const void* q, const int64_t* q_strides,
                          const void* k, const int64_t* k_strides,
                          const void* v, const int64_t* v_strides,
                          int64_t batch, int64_t query_tokens, int64_t key_tokens,
                          int64_t heads, int64_t head_dim, double scale, double beta,
                          int64_t local_blocks, int64_t kv_sink_tokens,
                          int64_t query_sink_tokens, void* out, int32_t* counts, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SOL_ATTN_AMD_H */
