// Structures shared by the host planner/launcher and the gfx950 kernels.
//
// A decode step is cut into work items.  A segment is either a run of pages
// shared by several sequences (a tree-shared prefix, the CoW sharing
// TreeState::fork creates, crates/dendrite-core/src/tree/state.rs:49-84) or
// one sequence's private tail; an item is one chunk of a segment's pages, one
// KV head and a block of the segment's query rows.  Every item writes one
// partial attention state (O normalised, log2-sum-exp) per query row into the
// workspace; the merge kernel combines the partial states of each
// (sequence, query head) by log-sum-exp into the output.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include "dendrite_hip.h"

#if defined(__HIPCC__)
#define DH_HOST_DEVICE __host__ __device__
#else
#define DH_HOST_DEVICE
#endif

namespace dh {

constexpr int kPageSize = 16;       // tokens per page (dendrite-ffi flashinfer/mod.rs:14)
constexpr int kWaves = 4;           // wave64s per workgroup
constexpr int kTileRows = 16;       // query rows of one MFMA tile
constexpr int kWaveRows = 16;       // rows of a wave item: one tile, one wave
constexpr int kGroupMaxPages = 512; // pages of one group item (LDS page-id list)
constexpr int kPrefillMaxPages = 2048;  // pages of one prefill item (its LDS page-id list)
constexpr int kWaveIdRegs = 4;      // wave items hold <= 256 page ids in registers
// Row tiles per wave of a group item: pages staged by direct global->LDS
// loads (16-bit KV; FP8 / MXFP8 at head_dim 128 and 256, converted to bf16
// in LDS) use two (one at head_dim 256, for registers); FP8 / MXFP8 pages at
// head_dim 64 (staged through registers) one.  A group item has
// kWaves * tiles * 16 rows.
constexpr int kGroupTiles8 = 1;
DH_HOST_DEVICE constexpr int group_tiles16(int head_dim) { return head_dim == 256 ? 1 : 2; }
DH_HOST_DEVICE constexpr int group_rows(bool fp8_kv, int head_dim) {
    return kWaves * ((fp8_kv && head_dim == 64) ? kGroupTiles8 : group_tiles16(head_dim)) * kTileRows;
}

// One attention work item (32 bytes): a run of pages of one segment chunk,
// one KV head and a block of query rows.
struct Item {
    uint32_t page_off;   // first page of the item in Plan::pages
    uint32_t npages;     // pages in the item (>= 1)
    uint32_t seq_off;    // first SeqSlot of the item's (segment, chunk)
    uint32_t row_begin;  // first row; row rho -> seq_local = rho / r, j = rho % r
    uint32_t nrows;      // rows in the item
    uint32_t kv_head;
    uint32_t flags;      // kItemTail: the item's last page is tail_seq's last page
    uint32_t tail_seq;
};
constexpr uint32_t kItemTail = 1u;
// kItemCausal (prefill): the item's rows see different numbers of tokens,
// row_len[row's virtual sequence] each; ItemLim bounds them.
constexpr uint32_t kItemCausal = 2u;

// Token range of a causal item: its pages start at token tok0 of the
// sequence; its rows see lmin .. lmax tokens (lmin > tok0, lmax <= the
// tokens its pages hold).
struct ItemLim {
    uint32_t tok0, lmin, lmax, pad;
};

// What one workgroup does: up to four wave items (one per wave, <= 16 rows
// each) or one group item (<= group_rows() rows: each wave owns a block of
// rows and all four waves read the same pages, staged once in LDS).
struct Task {
    uint32_t kind;       // kTaskWaves or kTaskGroup
    uint32_t first;      // first item
    uint32_t count;      // items (1 for a group task)
    uint32_t pad;
};
constexpr uint32_t kTaskWaves = 0u, kTaskGroup = 1u;

// Sequence of a (segment, chunk) and the partial-state slot it owns there.
struct SeqSlot {
    uint32_t seq;
    uint32_t slot;
};

// Per partial row: its log2-sum-exp of scaled scores and the power of two k
// its stored O carries (stored = O * 2^-k; k = 0 for fp32 partials).
struct PartialLse {
    float lse;
    float k;
};

// Workgroup b runs group item b when b < n_group_items; otherwise it runs the
// wave items n_group_items + 4 (b - n_group_items) + w, one per wave w, that
// exist (the planner emits its tasks in exactly this order).
struct AttendArgs {
    const Item* items;
    const uint32_t* pages;
    const SeqSlot* seqslots;
    const void* q;               // [B][Hq][D]
    const uint8_t* kv;           // pool data [P][2][Hkv][16][D]
    const void* scales;          // pool scale records (format dependent)
    const int32_t* last_page_len;
    void* ws_o;                  // [slots][Hq][D] normalised partial O: fp32 for f32 q,
                                 // else f16 scaled per row by 2^-k
    PartialLse* ws_lse;          // [slots][Hq]
    uint32_t hq, hkv, r, gqa_tiled;
    float scale_log2;            // |softmax scale| * log2(e), at least 2^-60 (> 0)
    uint32_t q_sign;             // XOR mask on the query elements' sign bits: a
                                 // negative scale is folded into the query, so the
                                 // kernels see scale_log2 > 0 and may order scaled
                                 // scores by raw ones
    uint32_t n_group_items, n_wave_items;
    // Prefill plans (kItemCausal items): tokens each virtual sequence sees,
    // and the group items' token ranges; null for decode plans.
    const uint32_t* row_len;
    const ItemLim* item_lim;
    // Prefill plans whose every row has one partial state: the items write
    // the normalised rows straight to out (no merge); null otherwise.
    void* out_direct;
    // Pages in the pool: a page id at or past it is read as page 0 (and, on
    // the CSR path, marks its sequence bad).  Plan ids are checked on the
    // host, so there this never fires.
    uint32_t page_limit;
    // Decode from device CSR tables (dh_decode_csr): items are derived on
    // the device from the tables (csr_item) instead of read from items;
    // null on the plan path.
    const int32_t* csr_indptr;
    const uint32_t* csr_slot_ptr;
    const uint32_t* csr_hdr;      // CsrHeader
    uint32_t* seq_bad;            // [B] set to 1 for a sequence with a bad page id
    uint32_t csr_nrb;             // row blocks of 16 per (chunk, kv head)
    // Cascade on the CSR path: per sequence, its leading pages read by group
    // items (bits 0..15) and the partial-state slots those take (bits
    // 16..31); its wave items cover the rest.  Null: no cascade.
    const uint32_t* csr_skip;
    // Direct decode plans: each wave task's items are the chunks of one
    // (sequence, KV head, row block); the workgroup merges its rows over the
    // sequence's slots (slot_ptr) into out itself.  0 / null otherwise.
    uint32_t wave_direct;
    const uint32_t* slot_ptr;
    void* out;
    // Last-page lengths carried in the kernel arguments (a host array at the
    // call, dh_decode_batch_host_lens): 4 bits per sequence, 0 meaning 16;
    // read when last_page_len is null and lpl_inline is 1.
    uint32_t lpl_inline;
    uint32_t lpl_nib[DH_HOST_LENS_MAX_BATCH / 8];
};

// What the CSR planning kernel leaves in the workspace for the attention
// and merge kernels of the same call.
struct CsrHeader {
    uint32_t chunk;        // pages per chunk of the wave items
    uint32_t n_items;      // wave items (0 when the tables exceed the workspace)
    uint32_t overflow;     // 1: more chunks than the workspace holds
    uint32_t n_chunks;     // partial-state slots used
    uint32_t n_group;      // group items (each a shared prefix's chunk, read once), first in the grid
    uint32_t group_chunk;  // pages per chunk of the group items
    uint32_t n_node_waves; // wave items of shared prefixes with few rows (items after the group items)
    uint32_t pad;
};

// Common-prefix scan of adjacent sequences (csr_lcp_kernel): boundary b
// (sequences b - 1 and b) is cut into kCsrLcpSlices slices of
// kCsrLcpSlice positions; each slice records its first mismatching position
// (or the boundary's cap, one page short of the shorter sequence, when none)
// in bits 0..15 and its first page id outside the pool before that in bits
// 16..31 (0xFFFF: none).  The common prefix is the minimum over the slices.
constexpr uint32_t kCsrLcpSlices = 16, kCsrLcpSlice = 512;
// Batches the CSR cascade is found for (one LDS entry per sequence), the
// pages a shared prefix must add to its parent's to form a node, and the
// node items (group and wave) a call may emit at most.
constexpr uint32_t kCsrCascadeMaxBatch = 512, kCsrMinShared = 8, kCsrMaxGroupItems = 4096;

// Inputs of the CSR planning kernel (one workgroup).
struct CsrPlanArgs {
    const int32_t* indptr;   // [B+1], device
    uint32_t batch;
    uint32_t per_chunk;      // wave items per chunk: hkv * row blocks
    uint32_t slot_cap;       // partial-state slots in the workspace (> batch)
    CsrHeader* hdr;
    uint32_t* slot_ptr;      // [B+1]
    uint32_t* seq_bad;       // [B]
    SeqSlot* seqslots;       // [slot_cap]
    // Cascade (null lcp: none): the common-prefix slices of csr_lcp_kernel,
    // the per-sequence skip words (AttendArgs::csr_skip) and the node items
    // written here (group items, then wave items), at most gcap of them;
    // group rows per item and the head shape they are cut by.
    const uint32_t* lcp;     // [B][kCsrLcpSlices]
    uint32_t* skip;          // [B]
    Item* gitems;            // [gcap]
    uint32_t gcap;
    uint32_t hkv, r, group_rows;
};

struct MergeArgs {
    const uint32_t* slot_ptr;    // [B+1] partial slots of sequence b
    const void* ws_o;            // as AttendArgs::ws_o
    const PartialLse* ws_lse;
    void* out;                   // [B][Hq][D]
    uint32_t batch, hq;
    uint32_t max_states;         // most partial states of a row (0: not known, up to 64)
    uint32_t uniform_slots;      // n > 0: sequence b's slots are b*n .. b*n+n-1 (no slot_ptr read)
    // CSR path (null otherwise): sequences marked bad get zeros, and the
    // call's status (DH_OK / DH_EINVAL / DH_ENOMEM) goes to *status.
    const uint32_t* seq_bad;
    const CsrHeader* csr_hdr;
    int32_t* status;
};

// Byte offset of the (page, plane, kv head) 16 x D block in the pool.
DH_HOST_DEVICE inline uint64_t plane_offset(uint32_t page, uint32_t plane, uint32_t head,
                                                 uint32_t hkv, uint32_t head_dim,
                                                 uint32_t elem_bytes) {
    return ((uint64_t(page) * 2u + plane) * hkv + head) * uint64_t(kPageSize) * head_dim *
           elem_bytes;
}

}  // namespace dh

// Kernel launchers (defined in decode_kernels.hip and write_kernels.hip).
// Return hipError_t as int.
extern "C++" {
namespace dh {
// Plan patches: words[idx[k]] = val[k] for k < n, in order, one small
// kernel on the stream (n <= kPatchWords).
constexpr uint32_t kPatchWords = 128;
int launch_plan_patch(uint32_t* words, uint32_t n, const uint32_t* idx, const uint32_t* val, void* stream);
int launch_write_pages(const uint32_t* ids, uint32_t n, const void* src, uint32_t src_dtype, uint8_t* data,
                       uint8_t* scales, uint32_t num_pages, uint32_t hkv, uint32_t d, uint32_t fmt,
                       void* stream);
// Device address of this GPU's static scratch array (decode_kernels.hip);
// call with the GPU current.  Returns hipError_t as int.
int static_scratch_address(void** out);
int launch_attend(const AttendArgs& a, uint32_t n_tasks, uint32_t q_dtype, uint32_t kv_format,
                  uint32_t head_dim, bool prefill, void* stream);
int launch_merge(const MergeArgs& a, uint32_t q_dtype, uint32_t head_dim, void* stream);
int launch_merge_states(const float* o_a, const float* lse_a, const float* o_b,
                        const float* lse_b, float* o_out, float* lse_out, uint32_t n_rows,
                        uint32_t head_dim, void* stream);
int launch_gather(const uint8_t* kv, const uint32_t* pages, uint32_t n_pages, uint32_t kv_head,
                  uint32_t hkv, uint32_t head_dim, uint32_t elem_bytes, uint8_t* out,
                  void* stream);
bool attend_supported(uint32_t q_dtype, uint32_t kv_format, uint32_t head_dim);
int launch_csr_plan(const CsrPlanArgs& p, void* stream);
int launch_csr_lcp(const int32_t* indptr, const int32_t* indices, uint32_t batch, uint32_t page_limit,
                   uint32_t* lcp, void* stream);
// Wave slots of the chip the CSR path schedules against (256 CUs x two
// workgroups x four waves), and its chunk sizes: 1 page up to what a wave
// item's page-id registers hold.
constexpr uint32_t kCsrWaveSlots = 2048;
constexpr uint32_t kCsrMinChunk = 1, kCsrMaxChunk = uint32_t(kWaveIdRegs) * 64;
}  // namespace dh
}
