/*
 * dendrite_hip.h — C ABI of the MI355X (gfx950) paged tree-decode attention
 * backend for Dendrite.
 *
 * Every entry point below replaces a piece of Dendrite's attention path; the
 * comment on each names the reference item it stands in for (paths are
 * relative to the Dendrite repository root).  Conventions:
 *
 *  - Plain C11: no C++ or torch types cross this boundary, nothing throws.
 *  - Every call returns a dh_status.  DH_OK is 0; on failure a description
 *    is kept in a thread-local buffer read by dh_last_error().
 *  - Device pointers are HIP device allocations owned by the caller (q, out,
 *    workspace, last_page_len).  The pool owns the paged KV memory.
 *  - Streams are hipStream_t passed as void* (NULL = the default stream).
 *    Calls are ordered by the stream the caller passes.
 *  - dh_decode_batch allocates nothing; the caller sizes the workspace with
 *    dh_plan_workspace_size.
 */
#ifndef DENDRITE_HIP_H
#define DENDRITE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- constants */

/* Tokens per page.  crates/dendrite-ffi/src/flashinfer/mod.rs:14 (PAGE_SIZE),
 * crates/dendrite-core/src/cache/mod.rs:61 (TOKENS_PER_BLOCK),
 * crates/dendrite-core/src/cache/paged.rs:41 (DEFAULT_PAGE_SIZE). */
#define DH_PAGE_SIZE 16u
/* crates/dendrite-ffi/src/flashinfer/mod.rs:17 (MAX_SEQ_LEN). */
#define DH_MAX_SEQ_LEN 131072u
/* BlockId::INVALID = u32::MAX, crates/dendrite-core/src/cache/block.rs:11.
 * A page-list entry holding it is skipped, as ReferenceBackend::decode skips
 * blocks it cannot find (attention/backend.rs:228-233). */
#define DH_INVALID_PAGE 0xFFFFFFFFu
/* NodeId::ROOT, crates/dendrite-core/src/tree/node.rs:12. */
#define DH_ROOT_NODE 0ull

/* ------------------------------------------------------------------ status */

/* Mirrors FfiError (crates/dendrite-ffi/src/error.rs:10-25) and the
 * DendriteError variants the path can raise (crates/dendrite-core/src/error.rs). */
typedef enum dh_status {
    DH_OK = 0,
    DH_EINVAL = 1,          /* FfiError::InvalidArgument / ShapeMismatch      */
    DH_ENOMEM = 2,          /* FfiError::AllocationFailed / OutOfMemory       */
    DH_EHIP = 3,            /* FfiError::CudaError (HIP runtime failure)      */
    DH_EUNSUPPORTED = 4,    /* FfiError::NotAvailable                         */
    DH_EINVALID_BLOCK = 5,  /* DendriteError::InvalidBlock                    */
    DH_EINVALID_NODE = 6,   /* DendriteError::InvalidNode                     */
    DH_ECACHE = 7           /* DendriteError::CacheError                      */
} dh_status;

/* Description of the last failure on the calling thread ("" if none). */
const char* dh_last_error(void);
/* Library version string. */
const char* dh_version(void);

/* ------------------------------------------------------------------ dtypes */

/* Query/output element type.  0 and 1 keep BatchDecodeConfig.dtype's encoding
 * (crates/dendrite-ffi/src/flashinfer/batch_decode.rs:18-19: 0=f16, 1=bf16). */
typedef enum dh_dtype {
    DH_DTYPE_F16 = 0,
    DH_DTYPE_BF16 = 1,
    DH_DTYPE_F32 = 2
} dh_dtype;

/* Paged KV element formats.  The FP8 formats follow
 * crates/dendrite-core/src/quantization/{mod.rs:47-82, fp8.rs:29-53}
 * with the OCP FP8 / MX v1.0 encodings. */
typedef enum dh_kv_format {
    DH_KV_F16 = 0,
    DH_KV_BF16 = 1,
    DH_KV_F32 = 2,
    /* E4M3 (OCP "FN": bias 7, max 448, S.1111.111 = NaN) with one fp32 scale
     * per (page, K|V, kv head): value = e4m3 * scale. */
    DH_KV_FP8_E4M3 = 3,
    /* MXFP8: E4M3 elements, one E8M0 scale (2^(e-127), e = 255 is NaN) per 32
     * consecutive elements along head_dim (QuantConfig.block_size = 32,
     * quantization/mod.rs:96-97). */
    DH_KV_MXFP8 = 4
} dh_kv_format;

/* Query head -> KV head mapping under grouped-query attention. */
typedef enum dh_gqa_mapping {
    /* head h reads KV head h % num_kv_heads: candle Tensor::repeat tiles the
     * KV heads, attention/backend.rs:245-252 (ReferenceBackend). */
    DH_GQA_TILED = 0,
    /* head h reads KV head h / (num_heads / num_kv_heads): HF-Llama repeat_kv,
     * crates/dendrite-core/src/model/layer.rs:321-340. */
    DH_GQA_INTERLEAVED = 1
} dh_gqa_mapping;

/* --------------------------------------------------------- attention config */

/* AttentionConfig, crates/dendrite-core/src/attention/backend.rs:17-28, plus
 * the dtype/mapping fields a device kernel needs. */
typedef struct dh_attn_config {
    uint32_t num_heads;       /* query heads                                   */
    uint32_t num_kv_heads;    /* KV heads; num_heads % num_kv_heads == 0       */
    uint32_t head_dim;        /* 64, 128 or 256 (flashinfer/mod.rs:20)         */
    float scale;              /* softmax scale, 1/sqrt(head_dim) by default;
                                 any finite value (0 gives uniform weights)   */
    uint32_t sliding_window;  /* 0 = None.  Accepted and ignored, as by every
                                 Dendrite backend (backend.rs:206-265 never
                                 reads it): attention spans all tokens.       */
    uint32_t gqa_mapping;     /* dh_gqa_mapping, DH_GQA_TILED by default       */
    uint32_t q_dtype;         /* dh_dtype of q and out (out dtype = q dtype)   */
    uint32_t kv_format;       /* dh_kv_format of the pool this config reads    */
} dh_attn_config;

/* AttentionConfig::new (backend.rs:32-40): scale = 1/sqrt(head_dim) computed
 * in f32, tiled GQA, bf16 queries, bf16 KV. */
dh_status dh_attn_config_init(dh_attn_config* cfg, uint32_t num_heads,
                              uint32_t num_kv_heads, uint32_t head_dim);
/* AttentionConfig::num_queries_per_kv (backend.rs:49-51). */
uint32_t dh_attn_config_num_queries_per_kv(const dh_attn_config* cfg);

/* ----------------------------------------------------------------- backend */

typedef struct dh_backend dh_backend;

/* Replaces dendrite-ffi's cudarc Device (crates/dendrite-ffi/src/cuda.rs:32-97)
 * and FlashInferBackend::new (attention/flashinfer.rs:211-237). */
dh_status dh_create(int device, dh_backend** out);
dh_status dh_destroy(dh_backend* backend);
/* cuda.rs:9-30: is_available / device_count. */
int dh_is_available(void);
dh_status dh_device_count(int* count);
/* cuda.rs:66-70 memory_info: free and total bytes of the backend's device. */
dh_status dh_memory_info(dh_backend* backend, size_t* free_bytes, size_t* total_bytes);
dh_status dh_synchronize(dh_backend* backend);

/* -------------------------------------------------------------- page pool */

typedef struct dh_pool dh_pool;

/* Device page pool: PagePool/Page (crates/dendrite-core/src/cache/paged.rs:
 * 54-308) with the page tensor [2][num_kv_heads][16][head_dim] (K plane, V
 * plane; paged.rs:57,90-94) laid out contiguously page after page:
 *   data   [num_pages][2][num_kv_heads][16][head_dim]  (kv_format element)
 *   scales DH_KV_FP8_E4M3: float   [num_pages][2][num_kv_heads]
 *          DH_KV_MXFP8   : uint8_t [num_pages][2][num_kv_heads][16][head_dim/32]
 * Memory is zero-filled at creation. */
dh_status dh_pool_create(dh_backend* backend, uint32_t num_pages,
                         uint32_t num_kv_heads, uint32_t head_dim,
                         uint32_t page_size, uint32_t kv_format, dh_pool** out);
dh_status dh_pool_destroy(dh_pool* pool);
/* Bytes of one page's data / scale record (0 for formats without scales). */
size_t dh_pool_page_bytes(const dh_pool* pool);
size_t dh_pool_scale_bytes(const dh_pool* pool);
uint32_t dh_pool_num_pages(const dh_pool* pool);
/* Device base pointers of the data and scale arrays (scales NULL if none). */
void* dh_pool_data(dh_pool* pool);
void* dh_pool_scales(dh_pool* pool);

/* Write tokens [tok_offset, tok_offset + n_tok) of one page from host memory.
 * k, v: [num_kv_heads][n_tok][head_dim] elements of the pool's format.
 * k_scale/v_scale: FP8_E4M3: float[num_kv_heads] (replaces the page's scale;
 * every FP8 block scale must be finite and > 0, else DH_EINVAL);
 * MXFP8: uint8[num_kv_heads][n_tok][head_dim/32]; ignored otherwise.
 * This is the device half of ReferenceBackend::append_kv/store_kv
 * (attention/backend.rs:285-301, 140-143) and Page::append (paged.rs:156-183).
 * Enqueued on `stream`; host buffers must stay valid until it completes. */
dh_status dh_pool_write_tokens(dh_pool* pool, uint32_t page_id, uint32_t tok_offset,
                               uint32_t n_tok, const void* k, const void* v,
                               const void* k_scale, const void* v_scale, void* stream);
/* Bulk upload of whole pages (data + scale records) from host memory:
 * page_ids[i] receives data[i] and scales[i] in the pool layout above.
 * Returns once the pages are written (the stream is synchronised).  The
 * upload goes through device staging memory of at most 256 MiB of pages;
 * the pool keeps up to 16 MiB of it from call to call and frees any larger
 * staging at the end of the call (uploads into one pool from several
 * threads take turns). */
dh_status dh_pool_write_pages(dh_pool* pool, const uint32_t* page_ids, uint32_t n,
                              const void* data, const void* scales, void* stream);
/* Quantise-on-write from device memory: page_ids[i] (device uint32[n]) of
 * the pool receives src[i] (device, 16-byte aligned,
 * [n][2][num_kv_heads][16][head_dim] of src_dtype, DH_DTYPE_*: K plane then
 * V plane; tokens past a partial page's length must be zero) in the pool's
 * format:
 *   F32 / BF16 / F16 : the value, converted with round to nearest even;
 *   FP8_E4M3         : scale = amax / 448 per (page, K|V, kv head), 1 if
 *                      amax = 0; element = E4M3 of x / scale, round to
 *                      nearest even, saturated to +-448 (fp8.rs:39-52);
 *   MXFP8            : per 32 consecutive elements along head_dim
 *                      (quantization/mod.rs:96-97) scale = 2^(floor(log2
 *                      amax) - 8) as E8M0 (2^-127 .. 2^127); element = E4M3
 *                      of x / scale, saturated.
 * Ids >= the pool size (INVALID included) are skipped: the ids live in device
 * memory, so the host cannot check them.  The device half of
 * ReferenceBackend::append_kv / store_kv (attention/backend.rs:285-301,
 * 140-143) for K/V already in HBM; the reference has no FP8 codec
 * (quantization/fp8.rs:29-53 states the ranges only).  Enqueued on `stream`;
 * allocates nothing. */
dh_status dh_pool_write_pages_device(dh_pool* pool, const uint32_t* page_ids, uint32_t n,
                                     const void* src, uint32_t src_dtype, void* stream);
/* Copy-on-write data copy src -> dst (all planes and scales).  The reference
 * leaves this as a TODO: crates/dendrite-core/src/cache/pool.rs:90. */
dh_status dh_pool_copy_page(dh_pool* pool, uint32_t src, uint32_t dst, void* stream);
/* Read one page (data, and scales if any) back to host memory (synchronous). */
dh_status dh_pool_read_page(dh_pool* pool, uint32_t page_id, void* data_out,
                            void* scales_out);

/* ------------------------------------------------------------ decode plan */

typedef struct dh_plan dh_plan;

/* Plan flags. */
#define DH_PLAN_FLAT 0u      /* every sequence reads its own pages            */
#define DH_PLAN_CASCADE 1u   /* pages shared by several sequences are read once
                                per step for all of them (tree-shared prefix) */

/* Tuning knobs of the work decomposition (all 0 = library defaults). */
typedef struct dh_plan_options {
    uint32_t shared_chunk_pages;   /* max pages of a shared segment per item   */
    uint32_t private_chunk_pages;  /* max pages of a private tail per item     */
    uint32_t target_items;         /* split chunks until about this many items */
    uint32_t direct;               /* DH_DIRECT_AUTO or DH_DIRECT_OFF          */
    uint32_t reserved[4];
} dh_plan_options;

/* dh_plan_options.direct: by default a decode plan in which no page run is
 * shared and every (sequence, KV head, block of 16 query rows) fits one
 * workgroup (its pages in at most four chunks, one per wave) is "direct":
 * each workgroup merges its waves' partial states itself and writes out, so
 * dh_decode_batch is one kernel launch.  DH_DIRECT_OFF plans it like any
 * other (chunks merged by the merge kernel). */
#define DH_DIRECT_AUTO 0u
#define DH_DIRECT_OFF 1u

/* Build the work decomposition of one decode step from host-side page lists
 * in CSR form (indices[indptr[b] .. indptr[b+1]) are sequence b's pages in
 * logical order, BlockTable::blocks(), cache/block_table.rs:83-85).  Entries
 * equal to DH_INVALID_PAGE are skipped; ids >= the pool size are DH_EINVAL.
 * With DH_PLAN_CASCADE a trie over the page-id sequences finds the runs of
 * pages shared by several sequences (the CoW prefixes TreeState::fork makes,
 * tree/state.rs:49-84); each run is attended once for all its sequences and
 * merged with each sequence's private tail by log-sum-exp.
 * Replaces BatchDecodeKernel::new (flashinfer/batch_decode.rs:31-54) and
 * CascadeAttention::new (flashinfer/cascade.rs:40-53): validation of head_dim
 * and num_heads % num_kv_heads happens here.  The plan is reusable for any
 * number of steps while the page lists keep their pages (the length of each
 * sequence's last page is a per-call input). */
dh_status dh_plan_create(dh_backend* backend, const dh_attn_config* cfg,
                         const dh_pool* pool, const uint32_t* indptr,
                         const uint32_t* indices, uint32_t batch_size,
                         uint32_t flags, const dh_plan_options* options,
                         dh_plan** out);
dh_status dh_plan_destroy(dh_plan* plan);

/* Events of one decode step for dh_plan_update. */
#define DH_PLAN_APPEND 0u        /* the sequence gained a page at the end      */
#define DH_PLAN_REPLACE_LAST 1u  /* its last page was replaced (copy-on-write) */

/* In-place update of a decode plan for the page-list changes one decode
 * step makes: the events of TreeState::append_token (tree/state.rs:87-113),
 * a new block on a block boundary (DH_PLAN_APPEND) and the copy-on-write of
 * a shared last block (DH_PLAN_REPLACE_LAST, the cow_dst of
 * dh_tree_append_token).  For k < n, event ops[k] applies page_ids[k] to
 * sequence seqs[k] (its index in the plan's batch), in order.  Each
 * sequence's last chunk is planned with room for 16 more pages; when every
 * event fits, the plan's device tables are patched by one small kernel per
 * 128 changed words on `stream` (ordered after earlier and before later
 * dh_decode_batch calls on that stream; a decode on another stream must not
 * overlap it) and *patched = 1.  When one does not fit (no room left, or a
 * sequence without pages) nothing changes, *patched = 0, and the caller
 * builds a new plan from the new page lists with dh_plan_create; forks (new
 * sequences, newly shared runs) always take a new plan.  The patched plan
 * reads exactly the pages the new lists hold and differs from a new plan
 * only in how each sequence's last pages are cut into items (results equal
 * within rounding).  Page ids must be inside the pool.  Not for prefill
 * plans (DH_EUNSUPPORTED).  After DH_EHIP the plan's device tables may be
 * partly patched: destroy it.  Updates of one plan must not overlap each
 * other on the host (the plan keeps host copies of its last chunks).  No counterpart in FlashInfer's plan / run
 * split (batch_decode.rs:31-101), which re-plans every step. */
dh_status dh_plan_update(dh_plan* plan, uint32_t n, const uint32_t* seqs, const uint32_t* ops,
                         const uint32_t* page_ids, void* stream, uint32_t* patched);
/* Workspace bytes dh_decode_batch needs with this plan
 * (cf. BatchDecodeKernel::workspace_size, batch_decode.rs:56-73). */
size_t dh_plan_workspace_size(const dh_plan* plan);

/* Plan statistics, for tests and benchmarks. */
typedef struct dh_plan_stats {
    uint32_t batch_size;
    uint32_t num_segments;        /* shared runs + private tails              */
    uint32_t num_shared_segments;
    uint32_t num_items;           /* attention work items                     */
    uint32_t num_tasks;           /* workgroups of the attention launch       */
    uint32_t num_group_items;     /* items whose pages four waves share       */
    uint32_t num_partials;        /* partial states per q head                */
    uint32_t direct;              /* 1: no merge launch (dh_plan_options.direct) */
    uint64_t unique_pages;        /* distinct pages read per step             */
    uint64_t page_reads;          /* pages read per step summed over items of
                                     one kv head (== unique_pages when every
                                     shared page is read once)               */
    uint64_t total_pages;         /* pages over all sequences (naive reads)   */
} dh_plan_stats;
dh_status dh_plan_get_stats(const dh_plan* plan, dh_plan_stats* stats);

/* One attention work item of a plan: pages[page_off .. +npages) of the plan's
 * page list, KV head kv_head, query rows row_begin .. +nrows of its
 * (segment, chunk).  Row rho belongs to sequence seqslots[seq_off + rho / r]
 * (r = num_heads / num_kv_heads), query head offset rho % r. */
typedef struct dh_plan_item {
    uint32_t page_off, npages, seq_off, row_begin, nrows, kv_head, flags, tail_seq;
} dh_plan_item;

/* Host-only planning for tests and tools: runs the same planner as
 * dh_plan_create on host inputs (no backend, no device) and copies out its
 * tables.  Call with NULL arrays to learn the sizes (*n_items, *n_pages,
 * *n_seqslots); seqslots receives (sequence, partial slot) pairs.  No
 * counterpart in the reference (a test export like dh_gather_debug). */
dh_status dh_plan_inspect(const dh_attn_config* cfg, uint32_t num_pool_pages,
                          const uint32_t* indptr, const uint32_t* indices,
                          uint32_t batch_size, uint32_t flags,
                          const dh_plan_options* options, dh_plan_stats* stats,
                          dh_plan_item* items, uint32_t* n_items,
                          uint32_t* pages, uint32_t* n_pages,
                          uint32_t* seqslots, uint32_t* n_seqslots);

/* Prefill plan (paged, causal).  Sequence b holds kv_len[b] tokens in its
 * pages (indptr / indices as for dh_plan_create, INVALID skipped; the last
 * page holds 1..16 of them) of which the last q_len[b] are the queries: rows
 * q_off[b] .. q_off[b] + q_len[b] of q and out (q_off = prefix sums of
 * q_len), each [num_heads][head_dim].  With causal != 0 query i of sequence
 * b sees tokens 0 .. kv_len[b] - q_len[b] + i (the bottom-right-aligned mask
 * of FA2 / FlashInfer); else all kv_len[b].  Run with dh_decode_batch (q /
 * out [sum q_len][num_heads][head_dim], last_page_len ignored).  Covers
 * ReferenceBackend::prefill (attention/backend.rs:163-204: q_len = kv_len,
 * causal) and BatchPrefillKernel::run (flashinfer/batch_prefill.rs:86-101,
 * K/V written to pages first); chunked prefill over a cached context is
 * q_len < kv_len.  bf16 / f16 queries (BatchPrefillConfig.dtype,
 * flashinfer/batch_prefill.rs:23), over FP8 / MXFP8 KV at head_dim 128 and
 * 256 as well (codes dequantised to the query's type in the kernel).  chunk_pages: KV pages per work item (0 = chosen from the work:
 * one item per block of queries when those fill the chip, else about 1024
 * items); at most about 2040 whatever is asked (an item's page-id list
 * holds 2048 entries), so longer contexts always take several items.
 * Host-side, synchronous. */
dh_status dh_plan_create_prefill(dh_backend* backend, const dh_attn_config* cfg,
                                 const dh_pool* pool, const uint32_t* indptr,
                                 const uint32_t* indices, const uint32_t* kv_len,
                                 const uint32_t* q_len, uint32_t batch_size, uint32_t causal,
                                 uint32_t chunk_pages, dh_plan** out);

/* ------------------------------------------------------------------ decode */

/* One decode step: out[b][h][:] = softmax(q[b][h] . K_b^T * scale) . V_b for
 * every sequence b of the plan, K_b/V_b being the tokens of b's pages in
 * order.  Semantics of ReferenceBackend::decode / decode_batch
 * (attention/backend.rs:206-283): GQA per cfg->gqa_mapping; a sequence with
 * no pages gets zeros (backend.rs:218-222, 235-238); INVALID ids are skipped.
 *   q, out        : device, [batch][num_heads][head_dim] of cfg->q_dtype
 *   last_page_len : device int32[batch] or NULL (all pages full).  Tokens in
 *                   each sequence's last page, 1..16.  0 is read as a full
 *                   page, the value PageTable::last_page_len reports for one
 *                   (cache/paged.rs:384-390).  Must be GPU-accessible memory
 *                   (a host array, e.g. from dh_tree_last_page_len, is copied
 *                   to the device first, or passed to
 *                   dh_decode_batch_host_lens); q, out, the workspace and it
 *                   are checked and a pageable host pointer is DH_EINVAL.
 *   workspace     : device, >= dh_plan_workspace_size(plan) bytes.
 * Replaces BatchDecodeKernel::run (batch_decode.rs:86-101) and
 * CascadeAttention::run (cascade.rs:84-101).  Allocates nothing. */
dh_status dh_decode_batch(dh_backend* backend, const dh_pool* pool,
                          const dh_plan* plan, const void* q,
                          const int32_t* last_page_len, void* out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Most sequences dh_decode_batch_host_lens takes. */
#define DH_HOST_LENS_MAX_BATCH 512u

/* dh_decode_batch with the last-page lengths read from host memory during
 * the call and carried to the kernels in their arguments (4 bits each): no
 * upload, no event, and the array may be reused as soon as the call
 * returns.  For callers whose lengths are host state that changes every
 * step, like the trait's decode_batch, which derives them from host block
 * tables (attention/backend.rs:80-85, 267-283).  last_page_len_host:
 * int32[batch] in host memory, or NULL (all pages full); values as for
 * dh_decode_batch (1..16; 0 or anything outside 1..16 reads as 16).
 * Plans of more than DH_HOST_LENS_MAX_BATCH sequences are DH_EUNSUPPORTED
 * (use dh_decode_batch).  Other arguments and results as dh_decode_batch;
 * allocates nothing. */
dh_status dh_decode_batch_host_lens(dh_backend* backend, const dh_pool* pool, const dh_plan* plan,
                                    const void* q, const int32_t* last_page_len_host, void* out,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the static scratch array behind dh_decode_batch_static (per GPU). */
#define DH_STATIC_WORKSPACE_BYTES (32u << 20)

/* dh_decode_batch that allocates nothing and takes no workspace: the partial
 * states go to a static device array of DH_STATIC_WORKSPACE_BYTES that the
 * library holds on every GPU it runs on until the process ends (its address
 * is looked up once per GPU by dh_create).  No counterpart in the reference:
 * for callers that cannot allocate device memory at decode time (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Plans whose dh_plan_workspace_size exceeds DH_STATIC_WORKSPACE_BYTES are
 * refused with DH_ENOMEM.  Every call on one GPU uses the same array, so
 * calls that overlap on one GPU (different streams or threads) race: order
 * them on one stream.  Nothing in the array needs clearing between calls
 * (every partial state a decode reads, it wrote).  Arguments and results as
 * dh_decode_batch. */
dh_status dh_decode_batch_static(dh_backend* backend, const dh_pool* pool, const dh_plan* plan,
                                 const void* q, const int32_t* last_page_len, void* out, void* stream);

/* ------------------------------------------------- decode from device CSR */

/* Workspace bytes dh_decode_csr needs for batch_size sequences whose page
 * tables hold at most max_total_pages entries together (indptr[batch] -
 * indptr[0] <= max_total_pages).  The size grows with batch_size and with
 * max_total_pages up to a cap (about two waves per wave slot of the chip,
 * 4 096 work items, in partial states, plus room for the shared prefixes'
 * chunks when the call may find them: one per 8 pages, at most 8 192), so
 * a workspace sized for a long context serves every shorter one.  Replaces
 * BatchDecodeKernel::workspace_size (flashinfer/batch_decode.rs:56-73). */
size_t dh_csr_workspace_size(const dh_attn_config* cfg, uint32_t batch_size, uint32_t max_total_pages);

/* One decode step from page tables that live on the device, read there on
 * every call: no plan, no host copy, no synchronisation.  The contract of
 * BatchDecodeKernel::run (flashinfer/batch_decode.rs:86-95):
 *   indices       : device int32[indptr[batch]], page ids in the pool
 *   indptr        : device int32[batch + 1], sequence b's pages are
 *                   indices[indptr[b] .. indptr[b+1])
 *   last_page_len : device int32[batch] or NULL, as for dh_decode_batch
 *   q, out        : device [batch][num_heads][head_dim] of cfg->q_dtype
 *   workspace     : device, >= dh_csr_workspace_size(cfg, batch, total) bytes
 *   status        : device int32 or NULL; the call's last kernel writes
 *                   DH_OK, DH_EINVAL (a page id outside the pool, a negative
 *                   indptr entry or one below its predecessor: those
 *                   sequences' outputs are zeros and no page outside the
 *                   pool is read) or DH_ENOMEM (the tables need more work
 *                   items than the workspace holds: every output is zeros).
 * Shared prefixes of consecutive sequences (what TreeState::fork
 * produces, tree/state.rs:49-84) are read once, as CascadeAttention
 * promises (flashinfer/cascade.rs:22-26): a first kernel compares every
 * pair of adjacent page lists; the planning kernel nests the common
 * prefixes into nodes (up to four levels, each adding at least 8 pages to
 * its parent's, runs of at least 16 query rows, batches of 2 to 512
 * sequences, 16-bit queries) whose pages are read once per KV head by
 * shared-prefix MFMA items (or multi-sequence wave items for short runs).
 * Every sequence's remaining pages are split into chunks of one page
 * count (the last chunk shorter), chosen on the device from the tables
 * for the earliest estimated end over the chip's wave slots, 1 to 256
 * pages; all partial states are merged by log-sum-exp.  A page id outside
 * the pool in a node's shared pages zeros every member.  Host checks
 * (returned synchronously): cfg and pool agree, the pointers are device
 * memory, the workspace holds at least batch + 1 chunks.  Four kernels on
 * `stream` (three without a cascade: f32 queries, one sequence, or more
 * than 512); allocates nothing. */
dh_status dh_decode_csr(dh_backend* backend, const dh_pool* pool, const dh_attn_config* cfg,
                        uint32_t batch_size, const void* q, const int32_t* indices,
                        const int32_t* indptr, const int32_t* last_page_len, void* out,
                        void* workspace, size_t workspace_bytes, int32_t* status, void* stream);

/* Stages of dh_decode_batch, for profiling: bit 0 = attention items,
 * bit 1 = log-sum-exp merge.  dh_decode_batch == stage mask 3.  Two kinds of
 * plan have no merge launch, and for them bit 0 alone runs the whole step
 * (attention and any merging, writing out) while bit 1 does nothing:
 *  - a direct decode plan (dh_plan_stats.direct = 1; DH_DIRECT_AUTO chooses
 *    one when nothing is shared and the sequences are short): each
 *    workgroup merges the states of its own rows before it ends;
 *  - a prefill plan in which every query row is one work item's (one
 *    partial state per row).
 * To profile the attention and the merge of a decode step apart, build its
 * plan with dh_plan_options.direct = DH_DIRECT_OFF. */
dh_status dh_decode_stages(dh_backend* backend, const dh_pool* pool,
                           const dh_plan* plan, const void* q,
                           const int32_t* last_page_len, void* out,
                           void* workspace, size_t workspace_bytes,
                           uint32_t stage_mask, void* stream);

/* ------------------------------------------------------------------- merge */

/* Element-wise log-sum-exp merge of two attention states
 * (merge_attention_outputs, crates/dendrite-ffi/src/flashinfer/cascade.rs:
 * 116-124), vectorised on the device:
 *   o_*  : device float[n_rows][head_dim], lse_* : device float[n_rows]
 *   m = max(lse_a, lse_b); o = (o_a e^(lse_a-m) + o_b e^(lse_b-m)) / sum;
 *   lse = m + ln(sum).
 * (-inf, -inf) yields o = 0, lse = -inf (the closed form would give NaN).
 * o_out/lse_out may alias the inputs. */
dh_status dh_merge_states(const float* o_a, const float* lse_a, const float* o_b,
                          const float* lse_b, float* o_out, float* lse_out,
                          uint32_t n_rows, uint32_t head_dim, void* stream);

/* ------------------------------------------------------------- test hooks */

/* The two entry points of this section have no counterpart in the reference
 * and replace nothing in its FFI: they expose pieces of the kernels to the
 * parity tests (page selection, FP8 / MXFP8 dequantisation).  The seeded
 * input generators of the tests and benchmarks are not part of this library
 * at all: they live in libdendrite_testdata.so (include/dendrite_testdata.h).
 *
 * Copy the K and V planes of kv head `kv_head` for the pages of a device page
 * list into out: [2][n_pages][16][head_dim] elements (K block then V block),
 * skipping DH_INVALID_PAGE entries (the output shrinks accordingly; *n_out
 * receives the pages copied).  Uses the decode kernels' page addressing, so a
 * byte-for-byte comparison with a host gather checks page selection. */
dh_status dh_gather_debug(const dh_pool* pool, const uint32_t* page_ids_host,
                          uint32_t n_pages, uint32_t kv_head, void* out_device,
                          uint32_t* n_out, void* stream);

/* The decode kernels' in-register E4M3 -> bf16 conversion on device `device`:
 * out[i] = bf16 bits of e4m3(codes[i]) * 2^(e8m0[i/4] - 127) (E8M0 255 = NaN).
 * n must be a multiple of 4; host buffers; synchronous.  For exhaustive tests
 * of the FP8 / MXFP8 dequantisation the kernels perform. */
dh_status dh_debug_e4m3_to_bf16(int device, const uint8_t* codes, const uint8_t* e8m0, uint32_t n,
                                uint16_t* out);

/* ------------------------------------------- host block model (CoW tables) */

/* Block pool with refcounts and a FIFO free list: BlockPool / KvCache,
 * crates/dendrite-core/src/cache/{pool.rs:10-103, mod.rs:61-143}, and Block
 * (cache/block.rs:36-109).  Thread-safe. */
typedef struct dh_block_pool dh_block_pool;
dh_status dh_block_pool_create(uint32_t max_blocks, uint32_t tokens_per_block,
                               dh_block_pool** out);
dh_status dh_block_pool_destroy(dh_block_pool* pool);
/* pool.rs:40-45: pops the front of the free list; DH_ENOMEM when empty. */
dh_status dh_block_pool_allocate(dh_block_pool* pool, uint32_t* block_id);
/* pool.rs:48-63: refcount - 1, back to the free list at 0. */
dh_status dh_block_pool_free(dh_block_pool* pool, uint32_t block_id);
/* pool.rs:66-73: refcount + 1. */
dh_status dh_block_pool_share(dh_block_pool* pool, uint32_t block_id);
/* pool.rs:76-97: unshared -> same id; shared -> a new id, old refcount - 1.
 * The reference copies no data (TODO pool.rs:90); callers pair a new id with
 * dh_pool_copy_page. */
dh_status dh_block_pool_copy_on_write(dh_block_pool* pool, uint32_t block_id,
                                      uint32_t* new_id);
uint32_t dh_block_pool_free_count(const dh_block_pool* pool);
uint32_t dh_block_pool_total(const dh_block_pool* pool);
/* Refcount of a block (0 for an id outside the pool). */
uint32_t dh_block_pool_refcount(const dh_block_pool* pool, uint32_t block_id);

/* Logical -> physical block table: BlockTable, cache/block_table.rs:10-109. */
typedef struct dh_block_table dh_block_table;
dh_status dh_block_table_create(uint32_t tokens_per_block, dh_block_table** out);
dh_status dh_block_table_destroy(dh_block_table* t);
uint32_t dh_block_table_num_blocks(const dh_block_table* t);
uint64_t dh_block_table_num_tokens(const dh_block_table* t);
/* get (block_table.rs:49-51): DH_EINVAL when out of range. */
dh_status dh_block_table_get(const dh_block_table* t, uint64_t logical_idx, uint32_t* id);
/* block_for_token (block_table.rs:54-57). */
dh_status dh_block_table_block_for_token(const dh_block_table* t, uint64_t token_pos,
                                         uint32_t* id);
dh_status dh_block_table_push(dh_block_table* t, uint32_t id);
/* set pads with DH_INVALID_PAGE (block_table.rs:65-70). */
dh_status dh_block_table_set(dh_block_table* t, uint64_t logical_idx, uint32_t id);
dh_status dh_block_table_set_num_tokens(dh_block_table* t, uint64_t n);
dh_status dh_block_table_add_tokens(dh_block_table* t, uint64_t n);
/* needs_new_block (block_table.rs:88-94). */
int dh_block_table_needs_new_block(const dh_block_table* t);
/* fork = independent copy (block_table.rs:97-103). */
dh_status dh_block_table_fork(const dh_block_table* t, dh_block_table** out);
dh_status dh_block_table_clear(dh_block_table* t);
/* Copies min(cap, num_blocks) ids into ids. */
uint32_t dh_block_table_blocks(const dh_block_table* t, uint32_t* ids, uint32_t cap);

/* Tree of CoW branches: TreeState / TreeNode, crates/dendrite-core/src/tree/
 * {state.rs:21-197, node.rs:43-146}.  Thread-safe. */
typedef struct dh_tree dh_tree;
typedef struct dh_node_info {
    uint64_t id;
    uint64_t parent;        /* DH_INVALID_NODE when the node is the root */
    uint64_t num_tokens;
    uint32_t num_children;
    uint32_t is_active;
} dh_node_info;
#define DH_INVALID_NODE 0xFFFFFFFFFFFFFFFFull
/* The tree keeps a reference to the block pool (which must outlive it). */
dh_status dh_tree_create(dh_block_pool* blocks, uint32_t tokens_per_block, dh_tree** out);
dh_status dh_tree_destroy(dh_tree* tree);
/* state.rs:49-84: child shares every valid block of the parent (refcount +1). */
dh_status dh_tree_fork(dh_tree* tree, uint64_t from_node, uint64_t* child,
                       uint64_t* depth, uint64_t* num_tokens);
/* state.rs:87-113: allocates a block on a block boundary, copy-on-writes the
 * last block.  When the copy-on-write gave the node a new block, *cow_src /
 * *cow_dst receive the old and new ids (else both DH_INVALID_PAGE), so the
 * caller can copy the page data with dh_pool_copy_page. */
dh_status dh_tree_append_token(dh_tree* tree, uint64_t node, uint32_t token,
                               uint32_t* cow_src, uint32_t* cow_dst);
/* state.rs:116-134 + gc 174-196. */
dh_status dh_tree_release(dh_tree* tree, uint64_t node);
/* state.rs:137-146: DH_EINVALID_NODE when absent. */
dh_status dh_tree_get_node(const dh_tree* tree, uint64_t node, dh_node_info* info);
/* state.rs:149-154: block ids of a node (copies min(cap, n)); *n = count. */
dh_status dh_tree_get_block_table(const dh_tree* tree, uint64_t node, uint32_t* ids,
                                  uint32_t cap, uint32_t* n);
/* Tokens generated at a node (node.rs:103-111); copies min(cap, n). */
dh_status dh_tree_get_tokens(const dh_tree* tree, uint64_t node, uint32_t* tokens,
                             uint32_t cap, uint32_t* n);
uint32_t dh_tree_num_nodes(const dh_tree* tree);
/* Tokens per block of the tree (TreeState's tokens_per_block, tree/state.rs:
 * 29-45; 0 for NULL).  The decode path reads 16-token pages, so the tree
 * entry points below take trees of DH_PAGE_SIZE-token blocks only. */
uint32_t dh_tree_tokens_per_block(const dh_tree* tree);

/* The cascade planner wired to TreeState: a decode plan over tree nodes (the
 * leaves being decoded), their page lists read from the tree's block tables
 * (TreeState::get_block_table, tree/state.rs:149-154) in one call, so the
 * caller assembles no CSR arrays.  Otherwise dh_plan_create with flags /
 * options; sequence i of the plan is nodes[i].  DH_EUNSUPPORTED for a tree
 * whose blocks are not DH_PAGE_SIZE tokens (a page holds 16 tokens). */
dh_status dh_plan_create_tree(dh_backend* backend, const dh_attn_config* cfg, const dh_pool* pool,
                              const dh_tree* tree, const uint64_t* nodes, uint32_t n, uint32_t flags,
                              const dh_plan_options* options, dh_plan** out);
/* last_page_len of each node for dh_decode_batch: its token count mod 16
 * (0 for a full last page, as PageTable::last_page_len reports it,
 * cache/paged.rs:384-390).  `out` is a HOST array of n entries:
 * dh_decode_batch reads last_page_len from device memory, so copy it there
 * first (hipMemcpyAsync on the decode's stream).  DH_EUNSUPPORTED for a tree
 * whose blocks are not DH_PAGE_SIZE tokens. */
dh_status dh_tree_last_page_len(const dh_tree* tree, const uint64_t* nodes, uint32_t n, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* DENDRITE_HIP_H */
