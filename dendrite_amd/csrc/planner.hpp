// Host-side decomposition of one decode step into attention work items.
#pragma once
#include <stdint.h>
#include <string>
#include <vector>
#include "dh_device.hpp"

namespace dh {

// Pages reserved after each sequence's last chunk, so a decode plan can take
// that many appended pages in place; no wave item holds more than
// kMaxItemPages (it keeps its page ids in registers, four per lane), no group
// item more than kGroupMaxPages (its LDS page-id list).
constexpr uint32_t kTailSlack = 16;
constexpr uint32_t kMaxItemPages = 256;

struct PlanInput {
    uint32_t batch = 0;
    const uint32_t* indptr = nullptr;   // [batch + 1]
    const uint32_t* indices = nullptr;  // [indptr[batch]]
    uint32_t num_pool_pages = 0;
    uint32_t hq = 0, hkv = 0;
    bool wave_items_only = false;       // f32: every item is a <= 16-row wave item
    uint32_t group_rows = 128;          // rows of a group item (group_rows())
    bool cascade = true;
    uint32_t shared_chunk_pages = 0;    // 0 = default
    uint32_t private_chunk_pages = 0;
    uint32_t target_items = 0;
    bool direct_ok = true;              // decode: a direct plan where one qualifies
};

struct HostPlan {
    std::vector<Task> tasks;
    std::vector<Item> items;
    std::vector<uint32_t> pages;
    std::vector<SeqSlot> seqslots;
    std::vector<uint32_t> slot_ptr;     // [batch + 1]
    uint32_t num_slots = 0;
    // Direct decode plan: wave task b holds the (at most kWaves) chunks of
    // one (sequence, KV head, row block), padded with empty items, and its
    // waves merge their own partial states (no merge kernel).
    bool direct = false;
    uint32_t num_group_items = 0;
    uint32_t num_wave_items = 0;
    uint32_t num_segments = 0;
    uint32_t num_shared_segments = 0;
    uint64_t unique_pages = 0;
    uint64_t page_reads = 0;            // pages read per KV head per step
    uint64_t total_pages = 0;
    // Prefill plans: tokens each virtual sequence (query) sees, and each
    // (causal) item's token range.
    std::vector<uint32_t> row_len;
    std::vector<ItemLim> item_lim;
    // Decode plans, per sequence b: the chunk holding its last page, for
    // in-place updates (appending a page, replacing the last page).  Its
    // pages are pages[tail_off[b] .. + tail_n[b]) and the entries up to
    // tail_cap[b] are reserved (DH_INVALID_PAGE); its items (one per KV head
    // and row block) are tail_items[tail_item_ptr[b] .. tail_item_ptr[b + 1]).
    // tail_n[b] = 0: the sequence has no pages.
    std::vector<uint32_t> tail_off, tail_n, tail_cap, tail_item_ptr, tail_items;
};

// Prefill: sequence b holds kv_len[b] tokens in its pages (CSR as for
// decode); its last q_len[b] tokens are queries, each a virtual sequence
// (rows of q / out in order).  Causal: query i sees kv_len - q_len + i + 1
// tokens, else all kv_len.
struct PrefillInput {
    uint32_t batch = 0;
    const uint32_t* indptr = nullptr;
    const uint32_t* indices = nullptr;
    const uint32_t* kv_len = nullptr;
    const uint32_t* q_len = nullptr;
    uint32_t num_pool_pages = 0;
    uint32_t hq = 0, hkv = 0;
    uint32_t group_rows = 128;
    bool causal = true;
    uint32_t chunk_pages = 0;           // 0 = chosen from the work
};

// Returns 0 on success, else a dh_status code with `err` set.
int build_plan(const PlanInput& in, HostPlan& out, std::string& err);
int build_prefill_plan(const PrefillInput& in, HostPlan& out, std::string& err);

}  // namespace dh
