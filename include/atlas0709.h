/*
 * atlas0709.h -- C ABI of the MI355X (gfx950) paged-KV tree path.
 *
 * One shared library (0709_amd/_lib/libatlas0709_hip.so) exports these entry
 * points.  Conventions shared by every call:
 *   - all pointers named *_dev are device (HBM) addresses; arrays named *_host
 *     are host memory that is copied into the kernel argument block;
 *   - memory is owned by the caller; no entry point allocates device memory;
 *   - work is enqueued on `stream` (a hipStream_t passed as void*) and the call
 *     returns without synchronising;
 *   - the return value is 0 on success, ATLAS_EINVAL for an argument error,
 *     ATLAS_EUNSUPPORTED for a configuration the kernels do not cover, and
 *     ATLAS_EHIP_BASE - hipError_t for a HIP runtime error.  atlas_last_error()
 *     returns a message for the last failing call on the calling thread.
 *
 * KV layouts.  A layer's K (or V) row for one token is `row_bytes` bytes
 * (num_kv_heads * head_dim * element size).  A physical slot id s starts at
 *     base + (s / page_size) * page_stride + (s % page_size) * token_stride
 * where base is the layer's K or V base address, and KV head h of the row at
 * h * head_stride from there (head_stride = head_dim * element size when the
 * row is contiguous).  This covers
 *   - FlashInfer NHD pages [pages, 2, page_size, Hkv, D] (V base = K base +
 *     page_size*token_stride, page_stride = 2*page_size*token_stride,
 *     contiguous rows),
 *   - FlashInfer HND pages [pages, 2, Hkv, page_size, D] (token_stride =
 *     head_dim * element size, head_stride = page_size * token_stride), and
 *   - SGLang's flat token pool [slots, Hkv, D] per layer (page_size = 1,
 *     separate K and V bases, page_stride = token_stride = row_bytes).
 * Entry points with head_bytes / head_stride arguments take rows split by KV
 * head: head_bytes (head_dim * element size) contiguous per head, head_stride
 * apart; head_stride = 0 or head_stride = head_bytes means contiguous rows.
 */
#ifndef ATLAS0709_H
#define ATLAS0709_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATLAS_OK 0
#define ATLAS_EINVAL (-1)
#define ATLAS_EUNSUPPORTED (-2)
#define ATLAS_EHIP_BASE (-1000)

/* Data types of KV / query / output elements. */
#define ATLAS_DTYPE_F16 0
#define ATLAS_DTYPE_BF16 1

/* Largest layer count one KV call carries in its argument block; larger pools
 * are processed in several launches by the same call. */
#define ATLAS_MAX_LAYERS_PER_LAUNCH 64
/* Largest item count for the *_host index variants (indices in kernarg). */
#define ATLAS_MAX_INLINE_ITEMS 64

const char* atlas_last_error(void);
int atlas_abi_version(void);

/* ------------------------------------------------------------------------
 * KV movement.  All three are HBM-bound 16-byte-vector gathers/scatters over
 * every layer in one launch.  row_bytes must be a multiple of 16 and every
 * base / stride a multiple of 16.
 * ---------------------------------------------------------------------- */

/* K[dst[i]] <- K[src[i]] and V[dst[i]] <- V[src[i]] for every layer.
 * Replaces SGLang MHATokenToKVPool.move_kv_cache(tgt_loc, src_loc) as called
 * by SGLangRoutePoolBridge._copy_kv_slots
 * (src/atlas_0709/flashinfer_paged/sglang_runtime.py:686-695), whose
 * semantics the reference pins as values[dst] = values[src]
 * (tests/test_tail_page_cow.py:14-16).  dst and src must be disjoint sets
 * (tail-page copy-on-write copies into freshly allocated pages). */
int atlas_kv_move_slots(const void* const* k_layers, const void* const* v_layers, int num_layers,
                        int64_t page_size, int64_t page_stride, int64_t token_stride,
                        int64_t row_bytes, const int64_t* dst_slots_dev,
                        const int64_t* src_slots_dev, int64_t n, void* stream);

/* Append: write dense per-layer source rows into slots.
 * K[slot_i] <- k_src_l[i], V[slot_i] <- v_src_l[i] for every layer l, where
 * slot_i = dst_slots_dev[i] when dst_slots_dev != NULL, else dst_start + i.
 * Source row i of layer l lives at k_src[l] + i * src_token_stride.
 * Replaces write_suffix_kv (src/atlas_0709/flashinfer_full_verify.py:1027-1042,
 * one layer, contiguous positions through the identity page table) and
 * SGLang set_kv_buffer as used by the Drafter decode
 * (src/atlas_0709/flashinfer_paged/sglang_page_attention.py:187-194). */
int atlas_kv_append(const void* const* k_layers, const void* const* v_layers, int num_layers,
                    int64_t page_size, int64_t page_stride, int64_t token_stride,
                    int64_t row_bytes, int64_t head_bytes, int64_t head_stride,
                    const void* const* k_src, const void* const* v_src,
                    int64_t src_token_stride, const int64_t* dst_slots_dev, int64_t dst_start,
                    int64_t n, void* stream);

/* Route-commit compaction through a page table.  For item i (request
 * item_req[i], or 0 when item_req is NULL) the logical positions src_pos[i]
 * and dst_pos[i] are mapped through that request's pages
 * kv_indices[kv_indptr[req] + pos / page_size] (identity when kv_indices is
 * NULL) and the row is copied for every layer.  The call is a gather followed
 * by a scatter, like the reference's clone-then-index_put: when some
 * destination equals another item's source it stages through `workspace_dev`
 * (needs n * 2 * num_layers * row_bytes bytes), otherwise it copies in place.
 * Replaces DirectFlashInferMaskedTreeVerifyBackend._commit_selected_path
 * (src/atlas_0709/target_runtime.py:873-920). */
int atlas_kv_commit_paged(const void* const* k_layers, const void* const* v_layers, int num_layers,
                          int64_t page_size, int64_t page_stride, int64_t token_stride,
                          int64_t row_bytes, int64_t head_bytes, int64_t head_stride,
                          const int32_t* kv_indptr_dev,
                          const int32_t* kv_indices_dev, const int32_t* item_req_dev,
                          const int64_t* src_pos_dev, const int64_t* dst_pos_dev, int64_t n,
                          int needs_staging, void* workspace_dev, size_t workspace_bytes,
                          void* stream);

/* Same as atlas_kv_commit_paged for up to ATLAS_MAX_INLINE_ITEMS items whose
 * request ids and positions are host arrays: they travel in the kernel
 * argument block, so the commit costs no host-to-device copy. */
int atlas_kv_commit_paged_host(const void* const* k_layers, const void* const* v_layers,
                               int num_layers, int64_t page_size, int64_t page_stride,
                               int64_t token_stride, int64_t row_bytes, int64_t head_bytes,
                               int64_t head_stride,
                               const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev,
                               const int32_t* item_req_host, const int64_t* src_pos_host,
                               const int64_t* dst_pos_host, int64_t n, void* stream);

/* ------------------------------------------------------------------------
 * Ancestor-masked paged tree / forest verify attention.
 * ---------------------------------------------------------------------- */

/* Work item of one attention workgroup (filled by the host planner).  The
 * per-request values after partial_row repeat what qo_indptr, kv_len,
 * mask_col_start and kv_indptr hold for `req`, so a workgroup reads everything
 * it needs to start streaming in one 64-byte load. */
typedef struct {
  int32_t req;          /* request index */
  int32_t kv_head;      /* KV head */
  int32_t row_start;    /* first packed query row (node * group + head_in_group) */
  int32_t num_rows;     /* packed rows handled (<= 256) */
  int32_t kv_start;     /* first key position (multiple of 64) */
  int32_t kv_end;       /* one past the last key position of this split */
  int32_t partial_row;  /* first row in the partial buffers, or -1 when the item
                           is the only split and writes the final output */
  int32_t qo_start;     /* qo_indptr[req] */
  int32_t qo_len;       /* qo_indptr[req + 1] - qo_indptr[req] */
  int32_t kv_len;       /* kv_len[req] */
  int32_t mask_col_start; /* mask_col_start[req] (tree mask), else 0 */
  int32_t page_offset;  /* kv_indptr[req] */
  int32_t pad[4];
} atlas_attn_work_t;

/* Merge item: combines `num_splits` partial states of one row block. */
typedef struct {
  int32_t req;
  int32_t kv_head;
  int32_t row_start;
  int32_t num_rows;
  int32_t partial_row;  /* partial row of split 0; split s row r lives at
                           partial_row + s * num_rows + r */
  int32_t num_splits;
  int32_t pad0;
  int32_t pad1;
} atlas_attn_merge_t;

/* First page-id window of every work item: window_dev[64 * i + l] = the page
 * id (from kv_indices_dev, at work[i].page_offset) of item i's page
 * work[i].kv_start / page_size + l, clamped to the item's last page, for
 * l < 64.  Run once per plan, after the work list and page table are in
 * place; atlas_tree_verify_attn then takes window_dev as page_window_dev
 * (NULL: the kernel reads the window from kv_indices after the work item).
 * With it a head_dim-128 workgroup requests its first page ids together with
 * its work item instead of one round trip later.  page_size must be a power
 * of two.  No counterpart in the reference: it is part of this library's
 * plan, as FlashInfer's plan keeps scheduling metadata of its own
 * (src/atlas_0709/flashinfer_full_verify.py:953-985 calls that plan). */
/* A plan's whole device set-up in one launch: the page windows of
 * atlas_attn_page_windows (window_dev NULL: none), read from src_indices_dev,
 * plus copies of the page table (n_indices int32 from src_indices_dev to
 * dst_indices_dev) and of the tree mask words (n_words int64 from
 * src_words_dev to dst_words_dev) into the plan's own buffers, which the
 * attention launches then read.  Sources and destinations must not overlap.
 * No counterpart in the reference, as atlas_attn_page_windows: part of this
 * library's plan (src/atlas_0709/flashinfer_full_verify.py:953-985 calls that
 * plan). */
int atlas_attn_plan_install(const atlas_attn_work_t* work_dev, int num_work, const int32_t* src_indices_dev,
                            int64_t n_indices, int32_t* dst_indices_dev, const int64_t* src_words_dev,
                            int64_t n_words, int64_t* dst_words_dev, int page_size, int32_t* window_dev,
                            void* stream);

int atlas_attn_page_windows(const atlas_attn_work_t* work_dev, int num_work,
                            const int32_t* kv_indices_dev, int page_size, int32_t* window_dev,
                            void* stream);

/* Host-side tree specification (no device work).  paths_host holds
 * num_paths routes of `depth` token ids each, row-major.  dedup != 0 builds
 * the prefix trie (one node per unique token prefix, numbered in creation
 * order, route by route, depth by depth), dedup == 0 one node per path
 * position.  Writes parents_host[node] (-1 for a root; capacity num_paths *
 * depth), route_nodes_host[route * depth + d] (may be NULL when dedup == 0)
 * and one packed buffer at out_host, in this order:
 *   token ids (int64, n), depths (int64, n),
 *   mask words (int64): n <= 64: word i = node i's ancestor-or-self bits;
 *     64 < n <= ATLAS_TREE_TILE_MAX_NODES: per node, one word per 64-key tile
 *     from prefix_len / 64 to (kv_len - 1) / 64 (ATLAS_MASK_TREE's wide
 *     layout); larger trees: none,
 *   int32: qo indptr {0, n}, kv indptr {0, pages}, last page length, the
 *     identity page table 0 .. pages - 1, a zero pad to an even count,
 *   the tree block of the dense mask: n x n bytes, [i][j] = 1 iff node j is
 *     an ancestor-or-self of node i.
 * info_host[0..7] = n, kv_len (prefix_len + n), pages, last page length,
 * mask words, words per node (tiles; 0 when n <= 64 or none), int32 count,
 * bytes written.  atlas_tree_spec_bytes() bounds the buffer for any paths of
 * that shape (-1 for an invalid shape); a smaller out_bytes than the tree
 * needs is refused with ATLAS_EINVAL.  Replaces the host work of
 * build_path_tree_tokens_from_paths, build_deduplicated_path_tree_tokens and
 * build_(deduplicated_)tree_spec_from_paths
 * (src/atlas_0709/flashinfer_full_verify.py:541-616, :655-739). */
#define ATLAS_TREE_TILE_MAX_NODES 1024
int64_t atlas_tree_spec_bytes(int32_t num_paths, int32_t depth, int64_t prefix_len, int32_t page_size);
int atlas_tree_spec_build(const int64_t* paths_host, int32_t num_paths, int32_t depth, int32_t dedup,
                          int64_t prefix_len, int32_t page_size, uint8_t* out_host, int64_t out_bytes,
                          int32_t* parents_host, int32_t* route_nodes_host, int64_t* info_host);
/* The spec's dense mask on the device from its tree block: mask_dev[i *
 * (prefix_len + n) + c] = 1 for c < prefix_len, block_dev[i * n + c -
 * prefix_len] otherwise (bytes, 0 or 1), one launch.  Replaces the dense
 * mask build of build_(deduplicated_)tree_spec_from_paths
 * (src/atlas_0709/flashinfer_full_verify.py:682-687, :719-724). */
int atlas_tree_mask_fill(const uint8_t* block_dev, int32_t n, int64_t prefix_len, uint8_t* mask_dev, void* stream);
/* The spec buffer of atlas_tree_spec_build moved to the device and its dense
 * mask filled, in one launch: the nbytes at spec_src (device memory, or
 * mapped pinned host memory: hipHostMalloc with hipHostMallocMapped and
 * hipHostMallocCoherent, through hipHostGetDevicePointer) are copied to
 * spec_dev, and mask_dev is filled as by atlas_tree_mask_fill from the tree
 * block, the spec's last n * n bytes, read at spec_src.  spec_src ==
 * spec_dev fills the mask only.  Both spec pointers 16-byte aligned.  Host
 * memory at spec_src must stay unchanged until the launch has completed.
 * Replaces the upload and the dense mask build of
 * build_(deduplicated_)tree_spec_from_paths
 * (src/atlas_0709/flashinfer_full_verify.py:682-687, :719-724). */
int atlas_tree_spec_upload(const uint8_t* spec_src, int64_t nbytes, int32_t n, int64_t prefix_len, uint8_t* spec_dev,
                           uint8_t* mask_dev, void* stream);

/* Mask modes. */
#define ATLAS_MASK_NONE 0   /* every key < kv_len visible */
#define ATLAS_MASK_TREE 1   /* keys < mask_col_start[req] visible; key p >= that
                               visible iff bit (p - start) of tree_mask[q]
                               (tree_mask_words == 1); with
                               tree_mask_words = W > 1 (wide trees), row q
                               holds W words at tree_mask[q * W ..], word j
                               covering the 64 keys of tile
                               start / 64 + j (bit b: key 64 (start / 64 + j)
                               + b, prefix keys set), and every work item
                               must start at a multiple of 64 keys */
#define ATLAS_MASK_CAUSAL 2 /* key p visible iff p <= kv_len - qo_len + q */

/* O = softmax(Q K^T * sm_scale + M) V over paged KV, GQA (num_qo_heads a
 * multiple of num_kv_heads), one launch for all requests plus a merge launch
 * when a row block is split along the keys.  q: [nnz, Hq, D]; kv_cache:
 * FlashInfer NHD pages [pages, 2, page_size, Hkv, D] or HND pages
 * [pages, 2, Hkv, page_size, D] addressed with the strides above (KV head h
 * of a token row at h * kv_head_stride); out: [nnz, Hq, D] in the input
 * dtype; lse (optional, may be
 * NULL): [nnz, Hq] fp32, natural-log log-sum-exp of the scaled scores.
 * workspace_dev holds the split partial states: partial_rows rows of D
 * 16-bit values in the output dtype (the normalised partial O, as FlashInfer
 * keeps its split-KV temporaries in the output type), then partial_rows fp32
 * base-2 LSEs: partial_rows * (2 * D + 4) bytes.  merge_partial_rows is the
 * count of partial rows the merge items reference (the plan's partial_rows,
 * passed with the merge list): a workspace holding fewer is refused with
 * ATLAS_EINVAL before any device work, and the kernels never write or read a
 * partial row the workspace does not hold.
 * Replaces FlashInfer BatchPrefillWithPagedKVCacheWrapper.plan/run with
 * causal=False and custom_mask as used by run_flashinfer_full_verify
 * (src/atlas_0709/flashinfer_full_verify.py:953-985, :1223). */
int atlas_tree_verify_attn(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                           const void* kv_cache, int64_t page_stride, int64_t kv_v_offset,
                           int64_t token_stride, int64_t kv_head_stride, const int32_t* qo_indptr_dev,
                           const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev,
                           const int32_t* kv_len_dev, int mask_mode,
                           const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev,
                           int tree_mask_words,
                           const atlas_attn_work_t* work_dev, int num_work,
                           const int32_t* page_window_dev,
                           const atlas_attn_merge_t* merge_dev, int num_merge,
                           int64_t merge_partial_rows, int max_rows_per_item,
                           int num_qo_heads, int num_kv_heads,
                           int head_dim, int page_size, float sm_scale, int dtype, void* out,
                           int64_t out_stride_token, int64_t out_stride_head, float* lse,
                           void* workspace_dev, size_t workspace_bytes, void* stream);

/* The same attention with the request's newest rows written first: for every
 * request, the K and V rows of its qo_len query tokens (append_k / append_v,
 * [token, Hkv, D] with the given strides in elements, token index = the
 * query row) go to its last qo_len key positions in the paged cache, inside
 * the attention launch, before any key tile is read.  One launch per layer
 * instead of write_suffix_kv followed by the attention
 * (src/atlas_0709/flashinfer_full_verify.py:1216-1222 writes with
 * write_suffix_kv, :1027-1042, then runs the wrapper, :1223).
 * head_dim 128 with a power-of-two page_size >= 16 (else ATLAS_EUNSUPPORTED).
 * The work list must give every (request, KV head) a single row block: the
 * items covering a request's newest positions write them for their KV head.
 * rope_cos / rope_sin (both or neither; [token, D] rows, stride in elements,
 * token index = the query row): q and append_k arrive before the rotary
 * embedding, which is applied in the launch with the rounding of the 16-bit
 * tensor ops q * cos + rotate_half(q) * sin that it replaces
 * (apply_rope_with_cos_sin, src/atlas_0709/flashinfer_full_verify.py:324-333,
 * called at :1213): the cache receives the rotated K rows bit for bit. */
int atlas_tree_verify_attn_append(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                                  const void* kv_cache, int64_t page_stride, int64_t kv_v_offset,
                                  int64_t token_stride, int64_t kv_head_stride, const int32_t* qo_indptr_dev,
                                  const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev,
                                  const int32_t* kv_len_dev, int mask_mode,
                                  const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev,
                                  int tree_mask_words,
                                  const atlas_attn_work_t* work_dev, int num_work,
                                  const int32_t* page_window_dev,
                                  const atlas_attn_merge_t* merge_dev, int num_merge,
                                  int64_t merge_partial_rows, int max_rows_per_item,
                                  int num_qo_heads, int num_kv_heads,
                                  int head_dim, int page_size, float sm_scale, int dtype, void* out,
                                  int64_t out_stride_token, int64_t out_stride_head, float* lse,
                                  void* workspace_dev, size_t workspace_bytes,
                                  const void* append_k, const void* append_v,
                                  int64_t append_stride_token, int64_t append_stride_head,
                                  const void* rope_cos, const void* rope_sin,
                                  int64_t rope_stride_token, void* stream);

/* Size of the device scratch array behind atlas_tree_verify_attn_noalloc:
 * 16 MiB per GPU, i.e. up to 64,527 partial rows at head_dim 128
 * (2 * 128 + 4 bytes each) or 127,100 at head_dim 64. */
#define ATLAS_ATTN_SCRATCH_BYTES 16777216

/* atlas_tree_verify_attn without a workspace: the split-KV partial states
 * (partial_rows rows, the count the plan produced; 0 when the plan has no
 * merge items) go to a device array of ATLAS_ATTN_SCRATCH_BYTES that the
 * library holds on every GPU it runs on until the process ends, so the call
 * allocates nothing and needs no workspace from the caller.  A plan whose
 * partial_rows * (2 * head_dim + 4) exceeds that size is rejected with
 * ATLAS_EINVAL, and so is a partial_rows below merge_partial_rows (checked,
 * like every buffer, before the device is touched).  Every call on one GPU
 * shares that GPU's array (nothing in it
 * needs to start at zero): calls that overlap on one GPU, on different
 * streams, race and must not be issued.  Results equal atlas_tree_verify_attn
 * with a workspace bit for bit (same kernels).
 * No counterpart in the reference: it exists for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid allocation). */
int atlas_tree_verify_attn_noalloc(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                                   const void* kv_cache, int64_t page_stride, int64_t kv_v_offset,
                                   int64_t token_stride, int64_t kv_head_stride, const int32_t* qo_indptr_dev,
                                   const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev,
                                   const int32_t* kv_len_dev, int mask_mode,
                                   const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev,
                                   int tree_mask_words,
                                   const atlas_attn_work_t* work_dev, int num_work,
                                   const int32_t* page_window_dev,
                                   const atlas_attn_merge_t* merge_dev, int num_merge,
                                   int64_t merge_partial_rows, int max_rows_per_item,
                                   int num_qo_heads, int num_kv_heads,
                                   int head_dim, int page_size, float sm_scale, int dtype, void* out,
                                   int64_t out_stride_token, int64_t out_stride_head, float* lse,
                                   int64_t partial_rows, void* stream);

/* ------------------------------------------------------------------------
 * Reachability prune and free-list return.
 * ---------------------------------------------------------------------- */

/* Mark-and-sweep over a page pool of num_pages pages held as bitmaps
 * (bit p of word p/32).  live_slots_dev lists slot ids of every live path (the
 * committed prefix and each retained route); their pages are marked live in
 * live_bitmap_dev (cleared first).  Every page set in owned_bitmap_dev but not
 * live is cleared from owned_bitmap_dev and written to free_pages_dev in
 * ascending order; the count goes to free_count_dev.
 * Replaces SGLangRoutePoolBridge.release_unreferenced_node_slots
 * (src/atlas_0709/flashinfer_paged/sglang_runtime.py:507-539):
 * releasable = sorted(owned - live). */
int atlas_prune_pages(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev, int64_t num_pages,
                      const int64_t* live_slots_dev, int64_t n_live_slots, int64_t page_size,
                      int64_t* free_pages_dev, int64_t* free_count_dev, void* stream);

/* One live slot path of atlas_prune_pages_paths: `len` slot ids at `slots`
 * (device memory). */
typedef struct {
  const int64_t* slots;
  int64_t len;
} atlas_slot_path_t;

#define ATLAS_PRUNE_MAX_PATHS 64

/* atlas_prune_pages with the live slots sampled from slot paths inside the
 * launch: path p (host array `paths`, copied into the launch arguments)
 * contributes its slots at indices 0, page_size, 2 page_size, ... and, when
 * bit p of last_slot_mask is set, its last slot -- one slot of every page of
 * a path laid out in whole pages (the committed prefix, and each retained
 * route with its last slot).  At most ATLAS_PRUNE_MAX_PATHS paths and
 * 524,288 pages (one workgroup's LDS bitmap); larger prunes return
 * ATLAS_EUNSUPPORTED and go through atlas_prune_pages.  Same result as
 * atlas_prune_pages over the concatenated samples; replaces the same
 * release_unreferenced_node_slots (sglang_runtime.py:507-539), whose live set
 * is the prefix plus every retained route's path. */
int atlas_prune_pages_paths(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev, int64_t num_pages,
                            const atlas_slot_path_t* paths, int num_paths, uint64_t last_slot_mask,
                            int64_t page_size, int64_t* free_pages_dev, int64_t* free_count_dev, void* stream);
/* A strided run of int64 values in device memory: src[0], src[stride], ...
 * (count of them). */
typedef struct {
  const int64_t* src;
  int64_t count;
  int64_t stride;
} atlas_i64_segment_t;
#define ATLAS_GATHER_MAX_SEGMENTS 32

/* atlas_prune_pages_paths, then the same launch copies the segments to out
 * as atlas_gather_i64 does (after its own released-page count is written,
 * so one of the segments may be free_count_dev): a prune and the read-back
 * of its results in one launch.  No counterpart in the reference: it ends
 * the prune of release_unreferenced_node_slots (sglang_runtime.py:507-539)
 * with the values the host needs next. */
int atlas_prune_pages_paths_gather(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev, int64_t num_pages,
                                   const atlas_slot_path_t* paths, int num_paths, uint64_t last_slot_mask,
                                   int64_t page_size, int64_t* free_pages_dev, int64_t* free_count_dev,
                                   const atlas_i64_segment_t* segments_host, int num_segments, int64_t* out,
                                   void* stream);

/* Set the owned bit of the pages of `n` slot ids (pages newly handed out). */
int atlas_mark_pages(uint32_t* bitmap_dev, int64_t num_pages, const int64_t* slots_dev, int64_t n,
                     int64_t page_size, void* stream);

/* Paged allocator slot assignment (the free list is a device int64 array of
 * page ids whose head the host advances by the number of pages consumed).
 * Decode: request i writes out[i] = last_loc[i] + 1 when seq_lens[i] - 1 is not
 * a multiple of page_size, else free_pages[j] * page_size where j counts the
 * earlier requests that also start a page.  Replaces SGLang
 * PagedTokenToKVPoolAllocator.alloc_decode as called by
 * SGLangRoutePoolBridge.allocate_decode_slots
 * (src/atlas_0709/flashinfer_paged/sglang_runtime.py:636-659). */
int atlas_alloc_decode_slots(const int64_t* seq_lens_dev, const int64_t* last_loc_dev,
                             const int64_t* free_pages_dev, int64_t page_size, int bs,
                             int64_t* out_dev, void* stream);

/* Extend: request i appends tokens prefix_lens[i] .. seq_lens[i]-1, first
 * continuing its partial tail page after last_loc[i], then opening pages from
 * the free list in request order; slots are packed in request order.
 * Replaces PagedTokenToKVPoolAllocator.alloc_extend as called by
 * SGLangRoutePoolBridge.allocate_extend_slots
 * (src/atlas_0709/flashinfer_paged/sglang_runtime.py:595-634). */
int atlas_alloc_extend_slots(const int64_t* prefix_lens_dev, const int64_t* seq_lens_dev,
                             const int64_t* last_loc_dev, const int64_t* free_pages_dev,
                             int64_t page_size, int bs, int64_t* out_dev, void* stream);

/* ------------------------------------------------------------------------
 * Paged metadata.
 * ---------------------------------------------------------------------- */

/* Compress concatenated token-slot paths into page tables.  Path b occupies
 * slots_dev[path_offsets_host[b] .. path_offsets_host[b+1]).  Writes
 * kv_page_indices (int32, one per page, page b's run starting at
 * page_offsets_host[b]) and, when validate != 0, sets *layout_ok_dev to 0 if
 * any page of any path is not page-aligned and contiguous (it must hold 1
 * before the call).  Replaces the per-route loop of
 * build_flashinfer_paged_kv_metadata
 * (src/atlas_0709/flashinfer_paged/paged_metadata.py:64-102). */
int atlas_paged_metadata(const int64_t* slots_dev, const int64_t* path_offsets_dev,
                         const int64_t* page_offsets_dev, int num_paths, int64_t total_pages,
                         int64_t page_size, int validate, int32_t* kv_page_indices_dev,
                         int32_t* layout_ok_dev, void* stream);

/* ------------------------------------------------------------------------
 * Frontier step of many requests in one launch.
 * ---------------------------------------------------------------------- */

/* The values of num_segments segments (at most ATLAS_GATHER_MAX_SEGMENTS, in
 * host memory; they travel in the launch's arguments) concatenated into out,
 * in one launch.  out may be mapped pinned host memory (hipHostMalloc with
 * hipHostMallocMapped and hipHostMallocCoherent, through
 * hipHostGetDevicePointer): the values are then on the host once an event
 * recorded after the launch has completed.  No counterpart in the reference:
 * it replaces the concatenation and device-to-host copy of a pool's small
 * results (released-page counts, prefix page starts, check words) that the
 * prune and commit read back. */
int atlas_gather_i64(const atlas_i64_segment_t* segments_host, int num_segments, int64_t* out, void* stream);

/* One active route of a frontier step (13 fields of 8 bytes).  The route's
 * new slot path is its current path with, when cow_tail > 0, the last
 * cow_tail slots replaced by the first slots of a fresh page (copy-on-write),
 * followed by its decode slot. */
typedef struct {
  const int64_t* path;    /* current slot path, prev_len int64 slots */
  int64_t prev_len;
  int64_t cow_tail;       /* 0, or 1 .. page_size-1 slots moved to a fresh page */
  int64_t cow_free_index; /* that page is free_pages[cow_free_index] */
  int64_t cow_offset;     /* its (dst, src) slot pairs go to cow_dst/cow_src[cow_offset ..] */
  int64_t new_free_index; /* >= 0: the decode slot opens page free_pages[new_free_index]
                             (required exactly when prev_len % page_size == 0);
                             < 0: it is the new path's last slot + 1 */
  int64_t flat_offset;    /* new path (prev_len + 1 slots) -> flat[flat_offset ..] */
  int64_t page_offset;    /* its page ids -> kv_page_indices[page_offset ..] (the
                             running sum of the earlier routes' page counts) */
  int64_t req_row;        /* request row that receives ... */
  int64_t write_start;    /* ... new path positions write_start .. prev_len */
  uint32_t* owned_bitmap; /* owned-page bitmap of the route's request (NULL: none) */
  int64_t group_first;    /* routes of the same request: group_first .. +group_count-1 */
  int64_t group_count;
} atlas_pool_frontier_route_t;

/* Bits of a route's check word (0: every check passed). */
#define ATLAS_FRONTIER_BAD_DESCRIPTOR 1  /* an index is out of range; the route was skipped */
#define ATLAS_FRONTIER_BAD_LAYOUT 2      /* a page of the new path is not page-aligned and contiguous */
#define ATLAS_FRONTIER_DUPLICATE_SLOT 4  /* another route of the request got the same decode slot */
#define ATLAS_FRONTIER_COW_OVERLAP 8     /* the copy-on-write page is a copy source of the request */
#define ATLAS_FRONTIER_MAX_HOST_ROUTES 24

/* The device half of SGLangRoutePoolBridge.prepare_frontier for the routes of
 * many requests that share one paged allocator, request-row pool and KV pool
 * (src/atlas_0709/flashinfer_paged/sglang_runtime.py:800-959 per request,
 * with allocate_decode_slots :636-659, the copy-on-write page choice of
 * _copy_partial_tail_pages_with_dirty_starts :708-798, the request-row
 * writes of _write_req_token_slice :1031-1092 and the page tables of
 * paged_metadata.py:64-102).  routes_dev holds num_routes descriptors, in
 * device memory.  Per route r it writes
 *   flat[flat_offset ..]      the new slot path,
 *   out_slots[r]              its decode slot,
 *   req_to_token[req_row * req_row_stride + p], p = write_start .. prev_len,
 *   kv_indptr[r + 1], kv_last_page_len[r], seq_lens[r] (kv_indptr[0] = 0),
 *   kv_page_indices[page_offset ..]  page id of each page of the new path,
 *   cow_dst/cow_src[cow_offset ..]   the slot pairs of its copy-on-write,
 * and sets the owned bits of its decode page and copy-on-write page, and
 * route_flags[r], its check word (ATLAS_FRONTIER_* bits; written for every
 * route, so nothing is cleared before the call).  The KV bytes of the copied
 * slots are not moved here (atlas_kv_move_slots). */
int atlas_pool_prepare_frontier(const atlas_pool_frontier_route_t* routes_dev, int num_routes,
                           const int64_t* free_pages_dev, int64_t num_free, int64_t page_size,
                           int64_t num_pages, int64_t* req_to_token_dev, int64_t req_rows,
                           int64_t req_row_stride, int64_t* flat_dev, int64_t flat_total,
                           int64_t* out_slots_dev, int64_t* cow_dst_dev, int64_t* cow_src_dev,
                           int64_t cow_total, int32_t* kv_indptr_dev, int32_t* kv_last_page_len_dev,
                           int32_t* seq_lens_dev, int32_t* kv_page_indices_dev, int64_t page_total,
                           int64_t* route_flags_dev, void* stream);

/* atlas_pool_prepare_frontier for up to ATLAS_FRONTIER_MAX_HOST_ROUTES routes
 * (one request's decode step) with the descriptors, tokens and route ids in
 * host memory: they travel in the launch's argument block, so no upload
 * precedes the launch.  It also writes the model inputs to batch_dev, five
 * runs of num_routes int64: tokens, sequence lengths (prev_len + 1),
 * positions (prev_len), request rows and route ids.  More routes return
 * ATLAS_EUNSUPPORTED.  No counterpart in the reference: the batch of one
 * that decode_frontier_one_token (sglang_runtime.py:1299-1346) runs. */
int atlas_pool_prepare_frontier_host(const atlas_pool_frontier_route_t* routes_host, const int64_t* tokens_host,
                                     const int64_t* route_ids_host, int num_routes, const int64_t* free_pages_dev,
                                     int64_t num_free, int64_t page_size, int64_t num_pages,
                                     int64_t* req_to_token_dev, int64_t req_rows, int64_t req_row_stride,
                                     int64_t* flat_dev, int64_t flat_total, int64_t* out_slots_dev,
                                     int64_t* cow_dst_dev, int64_t* cow_src_dev, int64_t cow_total,
                                     int32_t* kv_indptr_dev, int32_t* kv_last_page_len_dev, int32_t* seq_lens_dev,
                                     int32_t* kv_page_indices_dev, int64_t page_total, int64_t* route_flags_dev,
                                     int64_t* batch_dev, void* stream);

/* ------------------------------------------------------------------------
 * Route scoring.
 * ---------------------------------------------------------------------- */

/* out[i] = log_softmax(logits[row[i]])[token[i]] in fp32 for n gathers over
 * rows of `vocab` logits (dtype fp16, bf16, or ATLAS_DTYPE_F32 = 2): rows
 * 0 .. num_rows-1 of logits_dev, then rows num_rows .. num_rows+num_rows2-1
 * from logits2_dev (optional: num_rows2 = 0, NULL), so the verify logits and
 * the prefix logits of a Target verify are scored together.  One launch:
 * every row is read once, in chunks spread over the device, and its
 * log-sum-exp combined from the chunks in a fixed order (row_lse_dev, if not
 * NULL, receives it).  workspace_dev holds the chunk statistics and one
 * arrival counter per row: at least
 * atlas_gather_logprobs_workspace_bytes(num_rows, vocab) bytes, 16-byte
 * aligned, zero-filled before its first use; every call leaves it zero again
 * (calls sharing it must be stream-ordered).  Replaces the
 * two full-vocab log_softmax calls and the per-token gathers of
 * DirectFlashInferMaskedTreeVerifyBackend._score_routes
 * (src/atlas_0709/target_runtime.py:732-742). */
#define ATLAS_DTYPE_F32 2
int64_t atlas_gather_logprobs_workspace_bytes(int64_t num_rows, int64_t vocab);
int atlas_gather_logprobs(const void* logits_dev, int64_t row_stride, int64_t num_rows,
                          const void* logits2_dev, int64_t row_stride2, int64_t num_rows2,
                          int64_t vocab, int dtype, const int32_t* row_dev,
                          const int64_t* token_dev, int64_t n, float* row_lse_dev,
                          float* out_dev, void* workspace_dev, size_t workspace_bytes,
                          void* stream);

/* Route selection and commit positions of a Target verify, on the device (one
 * launch of one wave), so the commit can be queued behind the scoring without
 * a host round trip.  logprobs_dev holds the scoring launch's values in this
 * order: the first token of routes 0 .. num_routes - 1, then the remaining
 * depth - 1 tokens of route 0, of route 1, ...  Each value is rounded to the
 * logits dtype (rounding: ATLAS_ROUND_*), a route's score is the float64 sum
 * of its values from the left (with num_weights == depth, the float64 sum of
 * weights_host[t] * value_t instead); no operation is fused.  Policy
 * ATLAS_SELECT_TARGET_BEST selects the first route whose key (score,
 * draft_path_host[r], -route_ids_host[r]) is not exceeded by a later one
 * under tuple comparison (NaN equals nothing); ATLAS_SELECT_FIRST_ROUTE
 * selects route 0.  The selection falls back (commits nothing) when
 * has_first_threshold and its first value < first_threshold, or
 * has_path_threshold and its score < path_threshold.  Otherwise
 * commit_len_host[best] tokens are committed: for i < depth, src_dev[i] =
 * prefix_len + node_ids_host[best * depth + i] and dst_dev[i] = prefix_len + i
 * for i below the count, src_dev[i] = dst_dev[i] = prefix_len + i (a row
 * copied onto itself) past it.  result_dev[0] = the selected route's index,
 * result_dev[1] = the committed count (0 on fallback).  host_out (may be
 * NULL): device-accessible mapped host memory (hipHostMalloc with
 * hipHostMallocMapped, through hipHostGetDevicePointer) of num_routes * depth
 * floats plus two int32: the launch also writes the values there, rounded
 * to the logits dtype as the selection reads them, and the two result words
 * after them, visible to the host once the launch has completed
 * (an event recorded behind it), so no device-to-host copy is needed.
 * Limits: num_routes <=
 * ATLAS_SELECT_MAX_ROUTES, depth <= ATLAS_SELECT_MAX_DEPTH, num_routes *
 * depth <= ATLAS_SELECT_MAX_ENTRIES, node ids <= 32767.  Replaces the
 * selection of DirectFlashInferMaskedTreeVerifyBackend.verify_payloads
 * (src/atlas_0709/target_runtime.py:567-573 target_best and first_route,
 * :722-765 the scores, :754-760 the fallback thresholds, :873-920 the commit
 * positions); target_sample stays on the host. */
#define ATLAS_SELECT_MAX_ROUTES 64
#define ATLAS_SELECT_MAX_DEPTH 16
#define ATLAS_SELECT_MAX_ENTRIES 512
#define ATLAS_SELECT_TARGET_BEST 0
#define ATLAS_SELECT_FIRST_ROUTE 1
#define ATLAS_ROUND_NONE 0
#define ATLAS_ROUND_F16 1
#define ATLAS_ROUND_BF16 2
int atlas_route_select(const float* logprobs_dev, int num_routes, int depth, int policy, int rounding,
                       const double* weights_host, int num_weights, const double* draft_path_host,
                       const int64_t* route_ids_host, const int32_t* commit_len_host, const int32_t* node_ids_host,
                       int has_path_threshold, double path_threshold, int has_first_threshold,
                       double first_threshold, int64_t prefix_len, int64_t* src_dev, int64_t* dst_dev,
                       int32_t* result_dev, float* host_out, void* stream);

/* ------------------------------------------------------------------------
 * Drafter frontier: per-parent top-k, candidate order / selection, records.
 * ---------------------------------------------------------------------- */

#define ATLAS_MAX_FRONTIER_K 32
#define ATLAS_MAX_FRONTIER_CANDIDATES 4096

/* Candidate order / selection modes. */
#define ATLAS_FRONTIER_NONE (-1)          /* top-k only (records: order column -1) */
#define ATLAS_FRONTIER_ORDER 0            /* full stable order -> order_out */
#define ATLAS_FRONTIER_ORDER_BY_ROOT 1    /* the same with stage-1 root as first key */
#define ATLAS_FRONTIER_SELECT_GLOBAL 2    /* first num_selected of the order */
#define ATLAS_FRONTIER_SELECT_PER_ROOT 3  /* first num_selected of every root, roots ascending */
#define ATLAS_FRONTIER_PACK 4             /* records with a given selection */

/* Workspace bytes of atlas_frontier_topk for rows x vocab logits and k (any
 * contents; calls that share a workspace must be stream-ordered).  Negative
 * on bad arguments. */
int64_t atlas_frontier_workspace_bytes(int64_t rows, int64_t vocab, int k);

/* One frontier depth on the device, two launches, no host synchronisation.
 * For each logits row r ([rows, vocab] with row_stride elements; fp16, bf16
 * or fp32), the k tokens with the largest log_softmax(row) -- computed in
 * fp32 as (x - max) - log(sum exp(x - max)) and rounded to the logits dtype
 * -- in descending order, equal values by ascending token id:
 * token_logprobs_out[r, j] (logits dtype), token_ids_out[r, j].  Replaces
 * batch_parent_token_candidates' log_softmax + topk
 * (src/atlas_0709/flashinfer_paged/sampling.py:107-153).  With `proposal`
 * (fp32 Gumbel scores [rows, vocab], proposal_stride elements) the tokens are
 * the top-k of the proposal and their log-probs are gathered
 * (:139-153, the do_sample path).
 * With records_out ([rows * k + num_node_ids, 8] int64) the candidates of
 * build_pending_candidate_batch (frontier.py:127-185; parent_info_dev [rows, 3]:
 * route id, stage-1 root id, parent cumulative log-prob as float64 bits) are
 * written in the record layout of materialize_pending_candidate_batch
 * (frontier.py:188-265): kind 0, parent route, stage-1 root, token, rank in
 * parent, cumulative log-prob bits (parent + token log-prob in float64),
 * parent log-prob bits, selection order; then num_node_ids rows of kind 1
 * holding node_ids_dev.  select_mode ATLAS_FRONTIER_SELECT_GLOBAL / _PER_ROOT
 * selects as GlobalTopKSelection / PerStage1RootTopKSelection.select_indices
 * (frontier.py:58-124, utils.py:46-123) into selected_out and the order
 * column; ATLAS_FRONTIER_NONE leaves the order column -1.  k <= 32 and at most
 * 4096 candidates with records. */
int atlas_frontier_topk(const void* logits_dev, int64_t rows, int64_t vocab, int64_t row_stride,
                        int dtype, const float* proposal_dev, int64_t proposal_stride, int k,
                        const int64_t* parent_info_dev, int select_mode, int64_t num_selected,
                        const int64_t* node_ids_dev, int64_t num_node_ids,
                        void* token_logprobs_out, int64_t* token_ids_out, int64_t* records_out,
                        int64_t* parent_rows_out, int64_t* selected_out, void* workspace_dev,
                        size_t workspace_bytes, void* stream);

/* Order / select / pack a candidate batch given as six columns (element
 * strides in strides[0..5]: parent route, root, token, rank, cumulative
 * log-prob, parent log-prob).  The order is that of stable_candidate_order
 * (src/atlas_0709/flashinfer_paged/utils.py:46-83): cumulative log-prob
 * descending (NaN first, -0.0 == 0.0), then parent route, rank in parent and
 * token id ascending, then the original index; ORDER_BY_ROOT and
 * SELECT_PER_ROOT put the stage-1 root (ascending) first.
 * ORDER / ORDER_BY_ROOT: order_out[count] (the permutation).
 * SELECT_GLOBAL: global_topk_candidate_indices (:86-95) -> selected_out.
 * SELECT_PER_ROOT: per_root_topk_candidate_indices (:98-123), roots taken from
 * the candidates -> selected_out.  With records_out the candidates and the
 * selection order (or -1) are packed as materialize_pending_candidate_batch
 * does (frontier.py:188-265); PACK takes that selection from selected_in_dev
 * (num_selected_in entries; out-of-range entries are ignored).  count <= 4096. */
int atlas_candidate_select(const int64_t* parent_route_ids, const int64_t* stage1_root_ids,
                           const int64_t* pending_token_ids, const int64_t* ranks_in_parent,
                           const double* cumulative_logprobs, const double* parent_logprobs,
                           const int64_t* strides, int64_t count, int mode, int64_t num_selected,
                           const int64_t* selected_in_dev, int64_t num_selected_in,
                           const int64_t* node_ids_dev, int64_t num_node_ids, int64_t* order_out,
                           int64_t* selected_out, int64_t* records_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS0709_H */
