/* C ABI of libretrieve_amd.so: the MI355X (gfx950) scoring-and-selection hot path of
 * torchretrieve / SilverTorch.
 *
 * Conventions for every entry point:
 * - pointers are device pointers (HIP) unless stated; inputs are read-only and borrowed;
 *   outputs are caller-allocated; scratch comes from a caller-allocated `workspace` whose
 *   size the matching `*_workspace` function returns;
 * - work is enqueued on `stream` (a hipStream_t); no entry point synchronizes the host;
 * - the return value is 0 on success, else a status: 1 invalid argument (shape, size or
 *   range), 2 unsupported type/width, 3 a HIP call failed, 4 workspace too small;
 *   rt_last_error() then describes it;
 * - top-k results order by (score desc, item index asc): ties go to the lower item index.
 *   Rows with fewer than k candidates end in id -1 and the score sentinel (INT32_MIN for int32
 *   scores, -inf for float scores).
 */
#ifndef RETRIEVE_AMD_H_
#define RETRIEVE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* rt_stream_t; /* hipStream_t */

/* The message of the last failing call on this thread. */
const char* rt_last_error(void);

/* Exact int8 top-k over a full item table: int8 [B, D] queries x int8 [N, D] items, int32
 * dot products, top-k by (score desc, index asc) -> ids int64 [B, k], scores int32 [B, k].
 * D in {64, 128, 256, 512, 768, 1024}; 1 <= k <= 1024; N < 2**32 - 1.
 * `mask` (nullable): [B, mask_words] uint64, item d of row b passes iff bit 63 - d % 64 of
 * word d / 64 is set (SilverTorch's `filtering_bit_mask` order).
 * Replaces: SilverTorch's scorer + radix select for one cluster holding every item
 *   (silvertorch/silvertorch/ops/csrc/fork_search_cuda.cu:1256-1524, `st::search` with
 *   n_probe = n_lists = 1 and divisor_for_int8 = -1), and the int8 re-rank of
 *   retrieve/src/retrieve/modules/silvertorch.py:363-379 over all items. */
size_t rt_int8_scan_topk_workspace(int64_t B, int64_t N, int64_t D, int64_t k);
int rt_int8_scan_topk(const int8_t* queries, int64_t B, const int8_t* items, int64_t N,
                      int64_t D, int64_t k, const uint64_t* mask, int64_t mask_words,
                      int64_t* out_ids, int32_t* out_scores, void* workspace,
                      size_t workspace_bytes, rt_stream_t stream);

/* rt_int8_scan_topk without a workspace argument: the call allocates nothing (no hipMalloc,
 * no hipFree, no allocating library routine), so it suits callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid allocation. No
 * counterpart in the reference. Its scratch is a fixed 160 MiB device array per GPU, held
 * until the process ends. On a 256-CU part it holds the plan of up to 8192 queries at
 * k <= 224 and up to 4096 at k <= 480 (the candidate lists take 64 / 128 MiB whatever the
 * batch); a call whose plan needs more (k > 480 always) returns 1 (invalid argument) before
 * any launch, as does a null pointer. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams or threads) race and must be serialized by the caller. Same results
 * as rt_int8_scan_topk. */
int rt_int8_scan_topk_noalloc(const int8_t* queries, int64_t B, const int8_t* items, int64_t N,
                              int64_t D, int64_t k, const uint64_t* mask, int64_t mask_words,
                              int64_t* out_ids, int32_t* out_scores, rt_stream_t stream);

/* Dense (bf16 / fp16) full-scan top-k: queries [B, D] x items [N, D] of the same 16-bit type
 * (dtype 0 = bf16, 1 = fp16), fp32 accumulation on the matrix cores, top-k by
 * (score desc, index asc) -> ids int64 [B, k], scores float [B, k]. D in {32, 64, 128, 256,
 * 384, 512}; 1 <= k <= 1024. `mask` as for rt_int8_scan_topk.
 * Replaces: PostfilterKNN's torch.mm(q, E_t, out_dtype=fp32) + masked_topk / two_level_topk
 *   (retrieve/src/retrieve/modules/knn.py:62-76, retrieve/src/retrieve/functional.py:30-85)
 *   for LiNR V1's dense scores, fused so the [B, N] score matrix is never written. */
size_t rt_dense_scan_topk_workspace(int64_t B, int64_t N, int64_t D, int64_t k);
int rt_dense_scan_topk(const void* queries, int64_t B, const void* items, int64_t N, int64_t D,
                       int64_t k, int dtype, const uint64_t* mask, int64_t mask_words,
                       int64_t* out_ids, float* out_scores, void* workspace,
                       size_t workspace_bytes, rt_stream_t stream);

/* Large-batch form of rt_int8_scan_topk / rt_dense_scan_topk (same results): register-blocked
 * 32x32 MFMA tiles, 256 queries per workgroup held in registers, item tiles shared through
 * LDS. dtype 0 = int8 (int32 scores), 1 = bf16, 2 = fp16, 3 = fp32 (float scores). Rows of
 * 128, 256 or 512 bytes (int8 D in {128, 256, 512}; 16-bit D in {64, 128, 256}; fp32 D in
 * {32, 64, 128}). `row_bytes` of the
 * workspace function is D times the element size; `masked` != 0 sizes it for a call with a mask
 * (the mask is transposed into the workspace, ceil(N/64) x B words rounded up to 256 queries).
 * Replaces: the same reference paths as rt_int8_scan_topk / rt_dense_scan_topk at batches
 *   where they become a GEMM (B >= 128). */
size_t rt_blocked_scan_topk_workspace(int64_t B, int64_t N, int64_t row_bytes, int64_t k,
                                      int masked);
int rt_blocked_scan_topk(const void* queries, int64_t B, const void* items, int64_t N, int64_t D,
                         int64_t k, int dtype, const uint64_t* mask, int64_t mask_words,
                         int64_t* out_ids, void* out_scores, void* workspace,
                         size_t workspace_bytes, rt_stream_t stream);

/* Exact 1-bit Hamming top-k over a full code table: query_bits [B, W] x item_bits [N, W]
 * (uint64 words, bit b of word w = dimension 64 w + b), score = 64 W - 2 popcount(q ^ item),
 * top-k by (score desc, index asc) -> ids int64 [B, k], scores [B, k] (int32, or float when
 * score_f32 != 0). 1 <= W <= 16; 1 <= k <= 8192 (above 1024 the k-th score is found by
 * counting the 64 W + 1 scores and the ties at it by id bins: LiNR V3's candidate pools).
 * `mask` as for rt_int8_scan_topk. 512-bit codes (W = 8) from 8 queries on (k <= 1024) run on
 * the fp4 matrix cores (bits as e2m1 nibbles); `masked` of the workspace function as for
 * rt_blocked_scan_topk_workspace.
 * Replaces: the Triton full-scan kernel + torch.topk of
 *   retrieve/src/retrieve/ops/triton/oporp_1bit_match_topk.py:47-122, 217-234, 261-273
 *   (torch.ops.retrieve.oporp_1bit_match_topk_full). */
size_t rt_hamming_scan_topk_workspace(int64_t B, int64_t N, int64_t W, int64_t k, int masked);
int rt_hamming_scan_topk(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits,
                         int64_t N, int64_t W, int64_t k, const uint64_t* mask,
                         int64_t mask_words, int64_t* out_ids, void* out_scores, int score_f32,
                         void* workspace, size_t workspace_bytes, rt_stream_t stream);

/* Benchmark support (no counterpart in the reference): when enabled, every call brackets its
 * dominant kernel (the main scan) with a HIP event pair on its stream; collect() waits for
 * the recorded pairs, returns their summed milliseconds and count, and clears them. */
int rt_profile_enable(int on);
int rt_profile_collect(double* total_ms, int64_t* launches);

/* Measurement helper, no counterpart in the reference: the sustained rate of the matrix cores on
 * random operands (dtype 0: v_mfma_i32_32x32x32_i8, 1: v_mfma_f32_32x32x16_bf16), four
 * register-fed accumulator chains per wave, two waves per SIMD, `iters` steps per chain, and the
 * shader clock measured over the run (MHz). Sets *ops_per_s (int8 ops or bf16 flops per second).
 * Synchronizes the stream; allocates a small sink buffer for the duration of the call. */
int rt_mfma_ceiling(int dtype, int64_t iters, double* ops_per_s, double* clock_mhz,
                    rt_stream_t stream);

/* Measurement helper (no counterpart in the reference): the streaming-read rate of one kernel
 * over `bytes` at `data` (16-byte aligned): each 16-byte word read once per rep with
 * nontemporal loads, 64 workgroups a CU; a warm-up pass, then `reps` timed passes. Sets
 * *bytes_per_s. Synchronizes the stream; allocates a 4-byte sink for the call. */
int rt_read_ceiling(const void* data, int64_t bytes, int reps, double* bytes_per_s,
                    rt_stream_t stream);

/* ---- exact clause filter --------------------------------------------------------------
 *
 * Replaces the clause kernels behind torch.ops.retrieve.clause_mask / clause_mask_scores
 * (retrieve/src/retrieve/ops/triton/clause_mask.py:270-303; predicate functional.py:173-185)
 * and the exact payload filter of st::search (silvertorch/.../fork_filters.cuh:15-56).
 * item_attrs [N, C, A] of int16 / int32 / int64 (attr_bytes 2 / 4 / 8; -1 pads; the reference's
 * tables are int64); clause_is_reverse [C] 0/1; query_values [B, C, V]
 * int64, -1 pads (V == 1: the reference's [B, C], -1 = inactive clause). Clause c is active
 * for row b iff one of its V values is not -1; it matches iff an item value equals one of
 * them, XOR reverse[c]; an item passes iff every active clause matches. C <= 32.
 * mode 0: out = packed bits [B, ceil(N/64)] uint64, item d at bit 63 - d % 64 (the scans'
 *         mask layout), AND-ed with and_mask ([B, and_mask_words] words, same bit layout, e.g.
 *         a Bloom search's [B, n_bundles * 32]) when it is not null;
 * mode 1: out = [B, N] uint8 0/1;
 * mode 2: out = [B, N] float: scores[b, d] (contiguous [B, N]) where row b passes, -inf else. */
size_t rt_clause_filter_workspace(int64_t B, int64_t C, int64_t V);
int rt_clause_filter(const void* item_attrs, int attr_bytes, int64_t N, int64_t C, int64_t A,
                     const int8_t* clause_is_reverse, const int64_t* query_values, int64_t B,
                     int64_t V, int mode, const float* scores, const uint64_t* and_mask,
                     int64_t and_mask_words, void* out, void* workspace, size_t workspace_bytes,
                     rt_stream_t stream);

/* rt_int8_scan_topk (dtype 0) / rt_dense_scan_topk (dtype 1 bf16, 2 fp16) with the exact
 * clause filter of rt_clause_filter (same arguments and predicate) tested inside the scan: an
 * item is tested only where its composite beats its query's running bound, so no [B, N] mask is
 * written or read. `mask` (nullable, the scans' layout, e.g. a Bloom search's words) is AND-ed
 * in. Same results as the scan over rt_clause_filter's mode-0 bits AND mask; k <= 1024;
 * B <= 2^21.
 * Replaces: the exact clause post-check ANDed into the scan's mask
 *   (retrieve/src/retrieve/ops/triton/clause_mask.py:286-303 feeding
 *   retrieve/src/retrieve/functional.py:57-85) and st::search's per-doc exact filter inside its
 *   scorer (silvertorch/silvertorch/ops/csrc/fork_filters.cuh:15-41, called from
 *   fork_search_cuda.cu:918-1130). */
size_t rt_scan_topk_clauses_workspace(int64_t B, int64_t N, int64_t D, int64_t k, int64_t C,
                                      int64_t V);
int rt_scan_topk_clauses(const void* queries, int64_t B, const void* items, int64_t N, int64_t D,
                         int64_t k, int dtype, const uint64_t* mask, int64_t mask_words,
                         const void* item_attrs, int attr_bytes, int64_t C, int64_t A,
                         const int8_t* clause_is_reverse, const int64_t* query_values, int64_t V,
                         int64_t* out_ids, void* out_scores, void* workspace,
                         size_t workspace_bytes, rt_stream_t stream);

/* rt_blocked_scan_topk (same dtype codes and row sizes) with rt_scan_topk_clauses' exact clause
 * filter, for the items that pass `mask` (required here): the candidates that beat their
 * query's bound and pass the mask enter the lists, the clauses are tested where a list is
 * compacted and in the final merge (an entry that fails them is dropped), and the sampled bound
 * takes each lane's best over the mask, kept only when that item passes the clauses. Same
 * results as rt_blocked_scan_topk over rt_clause_filter's mode-0 bits AND mask. mask_t_stride
 * 0: `mask` is [B, mask_words] as above; > 0: it is already transposed, [mask_words, mask_t_stride]
 * (rt_bloom_search_t's layout: mask_words >= ceil(N/64) rows, mask_t_stride >= B rounded up to
 * 256), and the scan reads it as it is.
 * Replaces: as rt_scan_topk_clauses, at the batches of rt_blocked_scan_topk. */
size_t rt_blocked_scan_topk_clauses_workspace(int64_t B, int64_t N, int64_t row_bytes, int64_t k,
                                              int64_t C, int64_t V);
int rt_blocked_scan_topk_clauses(const void* queries, int64_t B, const void* items, int64_t N,
                                 int64_t D, int64_t k, int dtype, const uint64_t* mask,
                                 int64_t mask_words, int64_t mask_t_stride,
                                 const void* item_attrs, int attr_bytes,
                                 int64_t C, int64_t A, const int8_t* clause_is_reverse,
                                 const int64_t* query_values, int64_t V, int64_t* out_ids,
                                 void* out_scores, void* workspace, size_t workspace_bytes,
                                 rt_stream_t stream);

/* rt_hamming_scan_topk with the same fused clause filter, where the matrix-core scan takes the
 * batch (rt_hamming_scan_topk_clauses_fused(B, W, k) != 0: 512-bit codes, k <= 1024, the
 * batches of that kernel) and a mask is given; int32 scores, or float when score_f32. The mask
 * as for rt_blocked_scan_topk_clauses (mask_t_stride > 0: transposed).
 * Replaces: LiNR V3's filtered 1-bit shortlist (retrieve/src/retrieve/modules/linr.py:155-162,
 *   the clause mask of clause_compact feeding oporp_1bit_match_topk). */
int rt_hamming_scan_topk_clauses_fused(int64_t B, int64_t W, int64_t k);
size_t rt_hamming_scan_topk_clauses_workspace(int64_t B, int64_t N, int64_t W, int64_t k,
                                              int64_t C, int64_t V);
int rt_hamming_scan_topk_clauses(const uint64_t* query_bits, int64_t B, const uint64_t* item_bits,
                                 int64_t N, int64_t W, int64_t k, const uint64_t* mask,
                                 int64_t mask_words, int64_t mask_t_stride,
                                 const void* item_attrs, int attr_bytes,
                                 int64_t C, int64_t A, const int8_t* clause_is_reverse,
                                 const int64_t* query_values, int64_t V, int64_t* out_ids,
                                 void* out_scores, int score_f32, void* workspace,
                                 size_t workspace_bytes, rt_stream_t stream);

/* Packed mask [B, ceil(N/64)] (layout above) -> each row's set items in ascending order:
 * out_indices[b, 0:counts[b]] (int64, [B, N] buffer; the tail is not written), counts [B].
 * The compaction of torch.ops.retrieve.clause_compact
 * (retrieve/src/retrieve/ops/triton/clause_compact.py:174-187, _host.py:50-79). */
size_t rt_mask_compact_workspace(int64_t B, int64_t N);
int rt_mask_compact(const uint64_t* mask, int64_t B, int64_t N, int64_t* out_indices,
                    int64_t* counts, void* workspace, size_t workspace_bytes,
                    rt_stream_t stream);

/* [B, N] 0/1 bytes (a bool mask) -> packed words [B, ceil(N/64)] (layout above), the form the
 * scans take. Replaces: the boolean `mask` argument of PostfilterKNN.forward / masked_topk
 *   (retrieve/src/retrieve/modules/knn.py:68-76, functional.py:57-85) handed to a fused scan. */
int rt_pack_mask(const uint8_t* valid, int64_t B, int64_t N, uint64_t* words,
                 rt_stream_t stream);

/* ---- Bloom index (bit-sliced 2048-doc bundles) -----------------------------------------
 *
 * Layout (silvertorch/.../bloom_indexer.cpp:79-110): bundle beta (docs 2048 beta ..) is
 * w_beta = bundle_b_offsets[beta+1] - bundle_b_offsets[beta] bits per doc; position p of doc d
 * is bit 63 - d % 64 of word (bundle_b_offsets[beta] + p) * 32 + (d % 2048) / 64. A token
 * (feature id, value) sets the first k distinct murmur(id, value, seed) % w_beta over seeds
 * 0, 1, ... (MurmurHash3_x64_128 of the 16-byte key id || value, h1 ^ h2;
 * silvertorch/.../bloom_index_util.cuh:60-107, 185-208).
 * Features (the st:: build ops' jagged layout, retrieve/src/retrieve/ops/official/adapter.py:
 * 45-62): feature_ids int32 [C]; feature_offsets int64 [N * C + 1], the values of doc d,
 * feature c at feature_values[feature_offsets[d*C + c] .. feature_offsets[d*C + c + 1]). */

/* max_terms[beta] = max over the bundle's docs of the doc's value count (the upstream width is
 * (int64)((double)(max_terms * k) * b_multiplier), bloom_indexer.cpp:52-70). nb = ceil(N/2048). */
int rt_bloom_bundle_terms(const int64_t* feature_offsets, int64_t N, int64_t C, int64_t* max_terms,
                          rt_stream_t stream);

/* Writes every word of the index (words: bundle_b_offsets[nb] * 32 uint64). max_width = the
 * largest w_beta (<= 256); 1 <= k <= 10, k <= every nonzero w_beta.
 * Replaces: st::bloom_index_build / st::bloom_index_build_fixed
 *   (silvertorch/.../bloom_indexer.cpp:117-136, bloom_indexer_cuda.cu:291-344, 942-961). */
int rt_bloom_build(const int32_t* feature_ids, int64_t C, const int64_t* feature_offsets,
                   const int64_t* feature_values, int64_t N, const int64_t* bundle_b_offsets,
                   int64_t max_width, int64_t k, uint64_t* words, rt_stream_t stream);

/* Evaluates plan_count encoded plans (retrieve_amd/bloom.py: per plan 8 byte offsets
 * [ops, offsets, parameters, hashes] x [begin, end) into plan_data, data_bytes long) over
 * every column: a term holds for a doc iff the first k distinct (hash % w_beta) of its hash_k
 * stored hashes are all set (silvertorch/.../bloom_index_search_cuda.cu:305-349); AND / OR /
 * NOT / EMPTY as in :471-534. Outputs (either may be null): out_mask [plan_count, nb * 32]
 * words in the mask layout above, out_bool [plan_count, nb * 2048] 0/1 bytes. A malformed
 * plan yields no match. 1 <= k <= 10, 1 <= max_stack <= 64.
 * Replaces: st::bloom_index_search_batch(_prepared)
 *   (silvertorch/.../bloom_index_search.cpp:551-590, bloom_index_search_cuda.cu:1829-1856). */
size_t rt_bloom_search_workspace(int64_t data_bytes, int64_t plan_count);
int rt_bloom_search(const uint64_t* words, const int64_t* bundle_b_offsets, int64_t n_bundles,
                    const int64_t* plan_offsets, const int8_t* plan_data, int64_t data_bytes,
                    int64_t plan_count, int64_t max_stack, int64_t k, int64_t hash_k,
                    int64_t* out_mask, uint8_t* out_bool, void* workspace, size_t workspace_bytes,
                    rt_stream_t stream);

/* rt_bloom_search with the words written transposed: out_mask_t [nb * 32, out_t_stride], column c
 * of plan b at out_mask_t[c * out_t_stride + b] (out_t_stride >= plan_count; the entries past
 * plan_count are left as they were). The blocked scans take this layout as their mask directly
 * (rt_blocked_scan_topk_clauses, rt_hamming_scan_topk_clauses with mask_t_stride > 0) instead of
 * transposing [B, ceil(N/64)] words themselves.
 * Replaces: the same search as rt_bloom_search; the layout has no counterpart in the reference
 *   (its consumers take the row-major words). */
int rt_bloom_search_t(const uint64_t* words, const int64_t* bundle_b_offsets, int64_t n_bundles,
                      const int64_t* plan_offsets, const int8_t* plan_data, int64_t data_bytes,
                      int64_t plan_count, int64_t max_stack, int64_t k, int64_t hash_k,
                      uint64_t* out_mask_t, int64_t out_t_stride, void* workspace,
                      size_t workspace_bytes, rt_stream_t stream);

/* The search in two parts, so a batch's plans are compiled once (as the reference prepares them
 * once outside the forward, retrieve/src/retrieve/ops/official/adapter.py:184-236) and searched
 * any number of times. rt_bloom_compile writes every plan's folded program (or its stack-path /
 * no-match status) into `compiled` (rt_bloom_compiled_bytes(plan_count) bytes; the programs
 * depend on the plans, k, hash_k, max_stack and the width of bundle 0, nothing else of the
 * index). rt_bloom_search_compiled then searches, writing out_mask ([plan_count, nb * 32]) or
 * out_mask_t (rt_bloom_search_t's layout), exactly the words rt_bloom_search writes.
 * Clause mode (n_clauses in [1, 128]; 0: every plan runs its program): plans that are an AND of
 * clauses (a clause: an OR of terms, a term, or the NOT of either) over the batch's n_clauses
 * distinct clauses. Clause c is the OR of its terms, entries clause_ptr[c] .. clause_ptr[c + 1]
 * of clause_terms (4 words each: the term's program word pair, the index of its hash_k stored
 * hashes in plan_data as uint64 words, low and high). plan_desc[b]: bit 31 set for such a plan,
 * bits 12-30 its first entry in plan_refs, bits 0-11 its count; plan_refs: bits 0-14 a clause,
 * bit 15 its NOT. The column kernel evaluates each distinct clause once per column and such a
 * plan is the AND of its clauses' words; retrieve_amd/st.py's clause pass writes the tables.
 * plan_flags: bit 0 declares that every plan is a clause plan (the transposed words then leave
 * in contiguous runs: the kernel reuses its staging LDS to gather them); bit 1 that no plan takes
 * the stack evaluation (every status in `compiled` is a program or no-match): its launch is
 * skipped.
 * Replaces: st::bloom_index_search_batch_prepared (silvertorch/.../bloom_index_search.cpp:
 *   576-590) split at its plan preparation; no separate counterpart in the reference. */
size_t rt_bloom_compiled_bytes(int64_t plan_count);
int rt_bloom_compile(const int64_t* bundle_b_offsets, int64_t n_bundles,
                     const int64_t* plan_offsets, const int8_t* plan_data, int64_t data_bytes,
                     int64_t plan_count, int64_t max_stack, int64_t k, int64_t hash_k,
                     void* compiled, size_t compiled_bytes, rt_stream_t stream);
int rt_bloom_search_compiled(const uint64_t* words, const int64_t* bundle_b_offsets,
                             int64_t n_bundles, const int64_t* plan_offsets,
                             const int8_t* plan_data, int64_t data_bytes, int64_t plan_count,
                             int64_t max_stack, int64_t k, int64_t hash_k, const void* compiled,
                             size_t compiled_bytes, const uint32_t* clause_ptr,
                             const uint32_t* clause_terms, const uint32_t* plan_desc,
                             const uint32_t* plan_refs, int64_t n_clauses,
                             int64_t plan_flags, int64_t* out_mask, uint64_t* out_mask_t,
                             int64_t out_t_stride, rt_stream_t stream);

/* The index's row view: out_doc_bits[d] (uint64, n_docs <= n_bundles * 2048 of them) holds
 * document d's Bloom bits, position p at bit p, read from the bit-sliced bundles (layout above).
 * `width` is the index's bits per document (every bundle the same width, 1..64, as
 * st::bloom_index_build_fixed writes); a bundle of another width gives its documents all ones
 * (every probe passes them). Built once per index, beside it.
 * Replaces: no counterpart in the reference (whose search reads the bundles column-wise,
 *   silvertorch/.../bloom_index_search_cuda.cu:471-534); the bits are the same bundle words'
 *   (bloom_indexer.cpp:79-110). */
int rt_bloom_doc_bits(const uint64_t* words, const int64_t* bundle_b_offsets, int64_t n_bundles,
                      int64_t n_docs, int64_t width, uint64_t* out_doc_bits, rt_stream_t stream);

/* Probe tables: Bloom plans that are ANDs of at most 64 clauses (an OR of terms, a term, or the
 * NOT of either; none at all: EMPTY) as one uint64 array: words 0 .. plan_count hold each plan's
 * table offset in words from the array's start (plan b's table ends where b + 1's begins), then
 * the tables. A table: word 0 bit 0 set for a plan that matches nothing (a malformed one), bits
 * 1-31 its chunk count; word 1 the clauses in use (bit j: clause j); word 2 the negated
 * clauses; word 3 zero; then per chunk of 64 terms (the plan's terms in clause order) 64 words
 * of term position bits (bit p: position p for the index's width; all ones past the last
 * term) and 64 words, word j the chunk's term slots of clause j. A document with row bits f
 * passes when every clause holds a term whose bits f all has, XOR the clause's NOT.
 * retrieve_amd/st.py (probe_tables) writes them from rt_bloom_compile's programs and the plans'
 * op trees.
 * rt_bloom_probe_search: every plan (probe_tables, plan_count <= 65535) evaluated on every
 * document's row bits (rt_bloom_doc_bits): out_mask [plan_count, ceil(n_docs / 64)] in the mask
 * layout, the words the column search writes for documents below n_docs (bits at or past
 * n_docs are 0).
 * Replaces: st::bloom_index_search_batch_prepared (silvertorch/.../bloom_index_search.cpp:
 *   576-590) for such plans where every bundle has bundle 0's width; it is the per-document
 *   probe of rt_scan_topk_bloom_clauses over all documents. */
int rt_bloom_probe_search(const uint64_t* doc_bits, int64_t n_docs, const uint64_t* probe_tables,
                          int64_t plan_count, int64_t* out_mask, rt_stream_t stream);

/* rt_scan_topk_clauses with the Bloom pre-filter probed inside the scan instead of a mask: query
 * b's candidates (the items whose score beats its running bound) that pass the exact clauses
 * are tested against plan b's probe table (probe_tables, plan_count == B, above) on the
 * item's row bits (doc_bits, rt_bloom_doc_bits), a whole wave testing one candidate's terms at
 * once. No Bloom mask is written or read. Same results as rt_scan_topk_clauses with mask = the
 * Bloom search's words, when every bundle has the index's width. Over tables of 2^21 rows or
 * more the seed's bound is taken over the clauses alone; a query that ends with fewer than k
 * entries behind it (possible only where a plan rejects items its clauses pass) sets a flag and
 * a fallback pass without the bound recomputes the batch. Workspace:
 * rt_scan_topk_clauses_workspace.
 * Replaces: the Bloom pre-filter's mask (st::bloom_index_search_batch_prepared,
 *   silvertorch/.../bloom_index_search.cpp:576-590) feeding the filtered scorer with its exact
 *   post-check (fork_search_cuda.cu:1305-1342, fork_filters.cuh:15-41). */
int rt_scan_topk_bloom_clauses(const void* queries, int64_t B, const void* items, int64_t N,
                               int64_t D, int64_t k, int dtype, const uint64_t* doc_bits,
                               const uint64_t* probe_tables, int64_t plan_count,
                               const void* item_attrs, int attr_bytes, int64_t C, int64_t A,
                               const int8_t* clause_is_reverse, const int64_t* query_values,
                               int64_t V, int64_t* out_ids, void* out_scores, void* workspace,
                               size_t workspace_bytes, rt_stream_t stream);

/* The Bloom plans over the probed clusters' columns only: probed cluster i (row i / per_row of a
 * [rows, per_row] probe table) starts at doc position cluster_starts[i] and spans
 * column_counts_cumsum[i] - column_counts_cumsum[i - 1] columns (inclusive int32 cumsum) from
 * column cluster_starts[i] / 64; output word j of that span is row q's plan
 * (query_plan_index[q], or q) evaluated on its column, in the mask layout. Words from the device
 * total column_counts_cumsum[n_clusters - 1] up to max_columns are written 0; a plan index or
 * column outside the plans or the index gives 0. Plans and limits as rt_bloom_search.
 * Replaces: st::bloom_index_search_batch_return_partial_response[_prepared]
 *   (silvertorch/.../bloom_index_search.cpp:219-345, 561-601; bloom_index_search_cuda.cu:
 *   1739-1940). */
int rt_bloom_search_columns(const uint64_t* words, const int64_t* bundle_b_offsets,
                            int64_t n_bundles, const int64_t* plan_offsets,
                            const int8_t* plan_data, int64_t data_bytes, int64_t plan_count,
                            int64_t max_stack, int64_t k, int64_t hash_k,
                            const int64_t* cluster_starts, const int32_t* column_counts_cumsum,
                            int64_t n_clusters, int64_t clusters_per_row,
                            const int64_t* query_plan_index, int64_t max_columns,
                            int64_t* out_words, rt_stream_t stream);

/* ---- candidate lists ----------------------------------------------------------------
 *
 * Exact top-k over each query's own candidates: query row b against items
 * positive_indices[b, 0 : min(counts[b], P)] (int64 ids into the [N, D] table; ids outside
 * [0, N) are skipped), top-k by (score desc, item id asc) -> out_ids int64 [B, k] (-1 past the
 * row's candidates and, for float scores, where the score is not finite), out_scores [B, k].
 * kind 0 / 1 / 2: fp16 / bf16 / fp32 items [N, D] with float32 queries [B, D], fp32 dot,
 *   float scores;
 * kind 3: int8 items and queries [., D], int32 scores;
 * kind 4: bit codes of D uint64 words, score 64 D - 2 popcount(q ^ item), float scores.
 * Row bytes D * element size: a multiple of 16, at most 8192. 1 <= k <= 1024.
 * Replaces: torch.ops.retrieve.fused_masked_knn_topk
 *   (retrieve/src/retrieve/ops/triton/fused_masked_knn_topk.py:289-310; twin
 *   ops/reference/fused_masked_knn_topk.py:9-29), oporp_1bit_match_topk_indirect
 *   (ops/triton/oporp_1bit_match_topk.py:274-292; twin ops/reference/
 *   oporp_1bit_match_topk.py:29-41), and SilverTorch's int8 re-rank of given ids
 *   (retrieve/src/retrieve/modules/silvertorch.py:363-379). */
size_t rt_cand_topk_workspace(int64_t B, int64_t P, int64_t k);
int rt_cand_topk(const void* queries, int64_t B, const void* items, int64_t N, int64_t D, int kind,
                 const int64_t* positive_indices, int64_t P, const int64_t* counts, int64_t k,
                 int64_t* out_ids, void* out_scores, void* workspace, size_t workspace_bytes,
                 rt_stream_t stream);

/* Int8 re-rank of original ids: candidate c of row b (c < 0 or c >= N = padding, skipped) is
 * item_codes row item_rows[c] (a permutation, e.g. SilverTorch's inv_perm), scored as the float
 * (float(dot) * q_scales[b]) * global_scale[0]; the top min(k, P) by (score desc, id asc) ->
 * out_ids int64 / out_scores float32 [B, k], -1 / -inf past a row's candidates. Workspace as
 * rt_cand_topk_workspace(B, P, k).
 * Replaces: SilverTorch._forward_candidates (retrieve/src/retrieve/modules/silvertorch.py:
 *   363-379): the gather through inv_perm, the fp32 bmm of codes, the scaling and masked_topk. */
int rt_int8_rerank_topk(const int8_t* q_codes, const float* q_scales, int64_t B,
                        const int8_t* item_codes, int64_t N, int64_t D, const int64_t* item_rows,
                        const float* global_scale, const int64_t* candidate_ids, int64_t P,
                        const int64_t* counts, int64_t k, int64_t* out_ids, float* out_scores,
                        void* workspace, size_t workspace_bytes, rt_stream_t stream);

/* [1, N] float scores of one fp16 query [D] against the fp16 [D, N] item table (row k of the
 * table is dimension k of every item), accumulated as acc = fma(q[k], e[k, n], acc) for
 * k = 0 .. D-1 in fp32.
 * Replaces: torch.ops.retrieve.gemv_scores (retrieve/src/retrieve/ops/triton/gemv_scores.py:
 *   19-43), the B = 1 scorer of PostfilterKNN (retrieve/src/retrieve/modules/knn.py:62-66). */
int rt_gemv_scores(const uint16_t* query, const uint16_t* item_embs_t, int64_t D, int64_t N,
                   float* out, rt_stream_t stream);

/* ---- SilverTorch search ------------------------------------------------------------------- */

/* Per-row int8 quantization: abs_max = max(max |x|, 1e-8),
 * codes = clamp(rint(fp32(fp64(x) / fp64(abs_max)) * 127), -128, 127) (x float32 [rows, dim]);
 * scales[r] = abs_max / 127 when scale_div (quantize_int8), else abs_max * fp32(1/127)
 * (probe_prep).
 * Replaces: probe_prep's quantization (silvertorch/.../fork_search_cuda.cu:653-700) and
 *   retrieve/src/retrieve/indexing/quantize.py:9-18 (quantize_int8). */
int rt_quantize_int8_rows(const float* x, int64_t rows, int64_t dim, int8_t* codes,
                          float* scales, int scale_div, rt_stream_t stream);

/* Sign bits of float32 rows [rows, dim] (dim a multiple of 64) -> [rows, dim / 64] words, LSB
 * first: bit b of word w is x[r, 64 w + b] > 0 (NaN and -0 give 0).
 * Replaces: _pack_signs_to_int64 (retrieve/src/retrieve/indexing/quantize.py:63-72), the packing
 *   step of quantize_simhash_1bit / project_simhash_1bit_query and the Sign-OPORP projections
 *   (:99-173). */
/* quantize_int8_global (retrieve/src/retrieve/indexing/quantize.py:25-52): one scale for the
 * [rows, dim] float table, abs_max = max(max |x|, 1e-8) written to abs_max[0] (device), codes
 * clamp(rint(fp32(x / abs_max) * 127), -128, 127); row i of codes from row perm[i] of x when
 * perm (device, [rows]) is non-null. scratch4: 4 bytes of device memory. No host sync. */
int rt_quantize_int8_global(const float* x, int64_t rows, int64_t dim, const int64_t* perm,
                            int8_t* codes, float* abs_max, uint32_t* scratch4,
                            rt_stream_t stream);

int rt_pack_signs(const float* x, int64_t rows, int64_t dim, uint64_t* words,
                  rt_stream_t stream);

/* The exact clause filter over st::search's clause-major int32 slot layout (slots [R, N]; clause
 * c in rows clause_slots[c] .. clause_slots[c+1], -1 pads; query_values [B, C] int32, -1 =
 * inactive) -> packed bits [B, ceil(N/64)] as rt_clause_filter's mode 0, AND-ed with and_mask.
 * Replaces: the exact payload filter of st::search (silvertorch/.../fork_filters.cuh:15-56,
 *   fork_search_cuda.cu:957-1179). */
int rt_clause_slots_filter(const int32_t* slots, int64_t R, int64_t N, const int64_t* clause_slots,
                           int64_t C, const int8_t* clause_is_reverse, const int32_t* query_values,
                           int64_t B, const uint64_t* and_mask, int64_t and_mask_words,
                           uint64_t* out, rt_stream_t stream);

/* Top-k of SilverTorch's search over each row's probed clusters: row b's slots are the items of
 * clusters probe_ids[b, 0..n_probe) (sorted positions cluster_offsets[c] .. + cluster_sizes[c])
 * end to end, at most `width` of them; keys are the int32 dot of the int8 codes (divisor -1) or
 * fp16(float(dot) / divisor); top-k by (key desc, slot asc); items whose position's mask bit is
 * clear are skipped. Epilogue: out_ids = sort_perm[position], out_scores = (fp32(dot) * q_scale)
 * * global_scale[0] (fp16 path: score16 * ((q_scale * divisor) * global_scale[0])), -1 / -inf
 * pads. D (code bytes) a multiple of 16; n_probe <= 1024; 1 <= k <= 1024.
 * Replaces: st::search (silvertorch/.../fork_search_cuda.cu:1256-1524; schema
 *   fork_search.cpp:13-39) after its filter stage. */
size_t rt_ivf_search_workspace(int64_t B, int64_t width, int64_t k);
int rt_ivf_search(const int8_t* q_codes, const float* q_scales, int64_t B, const int8_t* item_codes,
                  int64_t N, int64_t D, const int64_t* probe_ids, int64_t n_probe,
                  const int64_t* cluster_offsets, const int64_t* cluster_sizes, int64_t n_lists,
                  int64_t width, const uint64_t* mask, int64_t mask_words, int64_t divisor,
                  const int64_t* sort_perm, int64_t n_perm, const float* global_scale, int64_t k,
                  int64_t* out_ids, float* out_scores, void* workspace, size_t workspace_bytes,
                  rt_stream_t stream);

/* rt_ivf_search with the reference's per-payload filters in place of a full-N mask: the probed
 * payloads' Bloom words in rt_bloom_search_columns' partial layout (entry b * n_probe + j for
 * probe j of row b: its docs from bit partial_first_offsets[e] of words
 * partial_counts_cumsum[e - 1] ...; null: no Bloom filter), and / or the exact recheck of the
 * probed docs in the slot layout (clause_slot_values [R, N] int32, clause c in rows
 * clause_slots[c] .. clause_slots[c + 1], clause_is_reverse [C] int8, query_clause_values [B, C]
 * int32 with -1 inactive; null: none; C <= 32). A doc is scored when every given filter passes.
 * Replaces: the payload filtering of st::search (fork_search_cuda.cu:1305-1342; the exact
 *   payloads of :918-1130 and fork_filters.cuh:15-41; the bloom partial payloads of
 *   bloom_index_search_cuda.cu:1945-2063). */
int rt_ivf_search_payload_filters(
    const int8_t* q_codes, const float* q_scales, int64_t B, const int8_t* item_codes, int64_t N,
    int64_t D, const int64_t* probe_ids, int64_t n_probe, const int64_t* cluster_offsets,
    const int64_t* cluster_sizes, int64_t n_lists, int64_t width,
    const int32_t* partial_counts_cumsum, const int8_t* partial_first_offsets,
    const uint64_t* partial_words, int64_t partial_entries, int64_t partial_n_words,
    const int32_t* clause_slot_values, int64_t R, const int64_t* clause_slots, int64_t C,
    const int8_t* clause_is_reverse, const int32_t* query_clause_values, int64_t divisor,
    const int64_t* sort_perm, int64_t n_perm, const float* global_scale, int64_t k,
    int64_t* out_ids, float* out_scores, void* workspace, size_t workspace_bytes,
    rt_stream_t stream);

/* SilverTorch's raw scorer: every probed doc's score in its slot of a [B, width] buffer.
 * Row b's probes j hold cluster_length[b, j] docs from cluster_offsets[cluster_ids[b, j]]
 * (n_offsets entries; an id outside them, or a cluster reaching outside the table, is empty);
 * the slots are every probe's full 32-doc warps in probe order, then every probe's remaining
 * docs in probe order, the first `width` of them. A written slot holds the score and the doc's
 * position (int32 out_indices); a slot past the row's docs or whose doc fails the filter holds the
 * score type's lowest value (INT32_MIN, fp16 -65504, bf16 / fp32 -max) and invalid_index.
 * elem: 0 int8 (queries and embeddings int8 [., D]), 1 bf16, 2 fp16, 3 fp32. Scores: int8 ->
 * int32 dot; int8 with divisor != -1 -> fp16(float(dot) / divisor); int8 with
 * per_embedding_scale (fp16 [N], taking precedence) -> fp16(float(fp16(dot)) / scale[doc]);
 * float rows -> the fp32-accumulated dot rounded to the row type; elem + 16 (bf16, fp16 or fp32
 * rows; an extension for this library's searches above k 1024) keeps the fp32 accumulator, fp32
 * scores. Filters (one at most): `mask`
 * [mask_rows, mask_words] in the mask layout over positions, row mask_index[b] (or b); or the
 * partial masks of rt_bloom_search_columns: entry e = mask_row * n_probe + j covers probe j's
 * docs from bit partial_first_offsets[e] of words partial_counts_cumsum[e - 1] ... D * element
 * size a multiple of 16, at most 8192 bytes; n_probe <= 1024; N < 2**31.
 * Replaces: st::fused_kmean_ann / st::fused_kmean_ann_with_partial_masks
 *   (silvertorch/.../fused_kmean_ann_cuda.cu:2126-2501; schemas fused_kmean_ann.cpp:420-460). */
int rt_fused_kmean_ann(const void* queries, const void* embeddings, int elem, int64_t B,
                       int64_t N, int64_t D, const int64_t* cluster_offsets, int64_t n_offsets,
                       const int64_t* cluster_ids, const int64_t* cluster_length,
                       int64_t n_probe, int64_t width, const uint64_t* mask, int64_t mask_rows,
                       int64_t mask_words, const int64_t* mask_index,
                       const int32_t* partial_counts_cumsum, const int8_t* partial_first_offsets,
                       const uint64_t* partial_words, int64_t partial_entries,
                       int64_t partial_n_words, int64_t divisor,
                       const uint16_t* per_embedding_scale, int64_t invalid_index,
                       void* out_scores, int32_t* out_indices, rt_stream_t stream);

/* The search epilogue alone, for a one-list search run as a full scan: ids [B, k] hold item
 * positions (-1 empty) and become sort_perm[position]; raw_dots [B, k] int32 -> out_scores. */
int rt_search_epilogue(int64_t* ids, const int32_t* raw_dots, float* out_scores, int64_t B,
                       int64_t k, const int64_t* sort_perm, int64_t n_perm, const float* q_scales,
                       const float* global_scale, rt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RETRIEVE_AMD_H_ */
