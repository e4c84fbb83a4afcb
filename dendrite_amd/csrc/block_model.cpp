// Host block model: the integer side of the path, restated in C++.
//   BlockPool / KvCache   crates/dendrite-core/src/cache/pool.rs:10-103, mod.rs:61-143
//   Block refcounts       crates/dendrite-core/src/cache/block.rs:36-109
//   BlockTable            crates/dendrite-core/src/cache/block_table.rs:10-109
//   TreeState / TreeNode  crates/dendrite-core/src/tree/state.rs:21-197, node.rs:43-146
// These produce the copy-on-write page lists the decode plan consumes.  The
// pool copies no page data itself (as in the reference, pool.rs:90); tree
// appends report the (old, new) ids of a copy-on-write so the caller can copy
// the device page with dh_pool_copy_page.
#include <deque>
#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

#include "dh_internal.hpp"

using dh::fail;

struct dh_block_pool {
    uint32_t tokens_per_block;
    std::vector<uint32_t> refcount;   // Block::refcount, 1 on allocation (block.rs:49-56)
    std::deque<uint32_t> free_list;   // FIFO (pool.rs:14, 40-45)
    mutable std::mutex mu;
};

struct dh_block_table {
    std::vector<uint32_t> blocks;
    uint64_t num_tokens = 0;
    uint32_t tokens_per_block = 16;
};

namespace {

dh_status pool_allocate(dh_block_pool* p, uint32_t* id) {
    if (p->free_list.empty()) return fail(DH_ENOMEM, "out of memory: no free blocks");
    *id = p->free_list.front();
    p->free_list.pop_front();
    p->refcount[*id] = 1;
    return DH_OK;
}

dh_status pool_free(dh_block_pool* p, uint32_t id) {
    if (id >= p->refcount.size()) return fail(DH_EINVALID_BLOCK, "invalid block id: %u", id);
    if (p->refcount[id] == 0) return fail(DH_EINVALID_BLOCK, "free of an unallocated block: %u", id);
    if (--p->refcount[id] == 0) p->free_list.push_back(id);
    return DH_OK;
}

dh_status pool_share(dh_block_pool* p, uint32_t id) {
    if (id >= p->refcount.size()) return fail(DH_EINVALID_BLOCK, "invalid block id: %u", id);
    p->refcount[id]++;
    return DH_OK;
}

dh_status pool_cow(dh_block_pool* p, uint32_t id, uint32_t* out) {
    if (id >= p->refcount.size()) return fail(DH_EINVALID_BLOCK, "invalid block id: %u", id);
    if (p->refcount[id] <= 1) {   // Block::is_shared is refcount > 1 (block.rs:81-83)
        *out = id;
        return DH_OK;
    }
    uint32_t nid;
    dh_status st = pool_allocate(p, &nid);
    if (st != DH_OK) return st;
    st = pool_free(p, id);
    if (st != DH_OK) return st;
    *out = nid;
    return DH_OK;
}

}  // namespace

struct TreeNodeRec {
    uint64_t id;
    uint64_t parent;           // DH_INVALID_NODE for the root
    dh_block_table table;
    std::vector<uint32_t> tokens;
    uint32_t num_children = 0;
    bool active = true;
};

struct dh_tree {
    dh_block_pool* pool;
    uint32_t tokens_per_block;
    uint64_t next_id = 1;      // NodeId::new counter (node.rs:23-29); ROOT = 0
    std::unordered_map<uint64_t, TreeNodeRec> nodes;
    mutable std::mutex mu;
};

extern "C" {

/* -------------------------------------------------------------- BlockPool */

dh_status dh_block_pool_create(uint32_t max_blocks, uint32_t tpb, dh_block_pool** out) {
    if (!out) return fail(DH_EINVAL, "out is NULL");
    *out = nullptr;
    if (tpb == 0) return fail(DH_EINVAL, "tokens_per_block must be positive");
    dh_block_pool* p = new (std::nothrow) dh_block_pool;
    if (!p) return fail(DH_ENOMEM, "out of host memory");
    p->tokens_per_block = tpb;
    p->refcount.assign(max_blocks, 0);
    for (uint32_t i = 0; i < max_blocks; ++i) p->free_list.push_back(i);
    *out = p;
    return DH_OK;
}

dh_status dh_block_pool_destroy(dh_block_pool* p) {
    delete p;
    return DH_OK;
}

dh_status dh_block_pool_allocate(dh_block_pool* p, uint32_t* id) {
    if (!p || !id) return fail(DH_EINVAL, "NULL argument");
    std::lock_guard<std::mutex> g(p->mu);
    return pool_allocate(p, id);
}

dh_status dh_block_pool_free(dh_block_pool* p, uint32_t id) {
    if (!p) return fail(DH_EINVAL, "pool is NULL");
    std::lock_guard<std::mutex> g(p->mu);
    return pool_free(p, id);
}

dh_status dh_block_pool_share(dh_block_pool* p, uint32_t id) {
    if (!p) return fail(DH_EINVAL, "pool is NULL");
    std::lock_guard<std::mutex> g(p->mu);
    return pool_share(p, id);
}

dh_status dh_block_pool_copy_on_write(dh_block_pool* p, uint32_t id, uint32_t* new_id) {
    if (!p || !new_id) return fail(DH_EINVAL, "NULL argument");
    std::lock_guard<std::mutex> g(p->mu);
    return pool_cow(p, id, new_id);
}

uint32_t dh_block_pool_free_count(const dh_block_pool* p) {
    if (!p) return 0;
    std::lock_guard<std::mutex> g(p->mu);
    return uint32_t(p->free_list.size());
}

uint32_t dh_block_pool_total(const dh_block_pool* p) { return p ? uint32_t(p->refcount.size()) : 0; }

uint32_t dh_block_pool_refcount(const dh_block_pool* p, uint32_t id) {
    if (!p) return 0;
    std::lock_guard<std::mutex> g(p->mu);
    return id < p->refcount.size() ? p->refcount[id] : 0;
}

/* ------------------------------------------------------------- BlockTable */

dh_status dh_block_table_create(uint32_t tpb, dh_block_table** out) {
    if (!out) return fail(DH_EINVAL, "out is NULL");
    if (tpb == 0) return fail(DH_EINVAL, "tokens_per_block must be positive");
    dh_block_table* t = new (std::nothrow) dh_block_table;
    if (!t) return fail(DH_ENOMEM, "out of host memory");
    t->tokens_per_block = tpb;
    *out = t;
    return DH_OK;
}

dh_status dh_block_table_destroy(dh_block_table* t) {
    delete t;
    return DH_OK;
}

uint32_t dh_block_table_num_blocks(const dh_block_table* t) { return t ? uint32_t(t->blocks.size()) : 0; }
uint64_t dh_block_table_num_tokens(const dh_block_table* t) { return t ? t->num_tokens : 0; }

dh_status dh_block_table_get(const dh_block_table* t, uint64_t idx, uint32_t* id) {
    if (!t || !id) return fail(DH_EINVAL, "NULL argument");
    if (idx >= t->blocks.size()) return fail(DH_EINVAL, "logical block %llu out of range", (unsigned long long)idx);
    *id = t->blocks[idx];
    return DH_OK;
}

dh_status dh_block_table_block_for_token(const dh_block_table* t, uint64_t pos, uint32_t* id) {
    if (!t) return fail(DH_EINVAL, "table is NULL");
    return dh_block_table_get(t, pos / t->tokens_per_block, id);
}

dh_status dh_block_table_push(dh_block_table* t, uint32_t id) {
    if (!t) return fail(DH_EINVAL, "table is NULL");
    t->blocks.push_back(id);
    return DH_OK;
}

dh_status dh_block_table_set(dh_block_table* t, uint64_t idx, uint32_t id) {
    if (!t) return fail(DH_EINVAL, "table is NULL");
    if (idx >= t->blocks.size()) t->blocks.resize(idx + 1, DH_INVALID_PAGE);
    t->blocks[idx] = id;
    return DH_OK;
}

dh_status dh_block_table_set_num_tokens(dh_block_table* t, uint64_t n) {
    if (!t) return fail(DH_EINVAL, "table is NULL");
    t->num_tokens = n;
    return DH_OK;
}

dh_status dh_block_table_add_tokens(dh_block_table* t, uint64_t n) {
    if (!t) return fail(DH_EINVAL, "table is NULL");
    t->num_tokens += n;
    return DH_OK;
}

static bool needs_new_block(const dh_block_table& t) {
    if (t.blocks.empty()) return true;
    return t.num_tokens % t.tokens_per_block == 0 && t.num_tokens > 0;
}

int dh_block_table_needs_new_block(const dh_block_table* t) { return t ? int(needs_new_block(*t)) : 0; }

dh_status dh_block_table_fork(const dh_block_table* t, dh_block_table** out) {
    if (!t || !out) return fail(DH_EINVAL, "NULL argument");
    dh_block_table* c = new (std::nothrow) dh_block_table(*t);
    if (!c) return fail(DH_ENOMEM, "out of host memory");
    *out = c;
    return DH_OK;
}

dh_status dh_block_table_clear(dh_block_table* t) {
    if (!t) return fail(DH_EINVAL, "table is NULL");
    t->blocks.clear();
    t->num_tokens = 0;
    return DH_OK;
}

uint32_t dh_block_table_blocks(const dh_block_table* t, uint32_t* ids, uint32_t cap) {
    if (!t) return 0;
    const uint32_t n = uint32_t(t->blocks.size());
    for (uint32_t i = 0; i < n && i < cap && ids; ++i) ids[i] = t->blocks[i];
    return n;
}

/* -------------------------------------------------------------- TreeState */

dh_status dh_tree_create(dh_block_pool* pool, uint32_t tpb, dh_tree** out) {
    if (!pool || !out) return fail(DH_EINVAL, "NULL argument");
    if (tpb == 0) return fail(DH_EINVAL, "tokens_per_block must be positive");
    dh_tree* t = new (std::nothrow) dh_tree;
    if (!t) return fail(DH_ENOMEM, "out of host memory");
    t->pool = pool;
    t->tokens_per_block = tpb;
    TreeNodeRec root;
    root.id = DH_ROOT_NODE;
    root.parent = DH_INVALID_NODE;
    root.table.tokens_per_block = tpb;
    t->nodes.emplace(DH_ROOT_NODE, std::move(root));
    *out = t;
    return DH_OK;
}

dh_status dh_tree_destroy(dh_tree* t) {
    delete t;
    return DH_OK;
}

dh_status dh_tree_fork(dh_tree* t, uint64_t from, uint64_t* child, uint64_t* depth, uint64_t* ntok) {
    if (!t) return fail(DH_EINVAL, "tree is NULL");
    std::lock_guard<std::mutex> g(t->mu);
    auto it = t->nodes.find(from);
    if (it == t->nodes.end()) return fail(DH_EINVALID_NODE, "invalid node id: %llu", (unsigned long long)from);
    TreeNodeRec c;
    c.id = t->next_id++;
    c.parent = from;
    c.table = it->second.table;   // BlockTable::fork, a Vec clone
    {
        std::lock_guard<std::mutex> pg(t->pool->mu);
        for (uint32_t b : c.table.blocks) {
            if (b == DH_INVALID_PAGE) continue;
            dh_status st = pool_share(t->pool, b);
            if (st != DH_OK) return st;
        }
    }
    it->second.num_children++;
    uint64_t d = 0;
    for (uint64_t cur = from;;) {
        auto n = t->nodes.find(cur);
        if (n == t->nodes.end() || n->second.parent == DH_INVALID_NODE) break;
        ++d;
        cur = n->second.parent;
    }
    const uint64_t id = c.id, tokens = c.table.num_tokens;
    t->nodes.emplace(id, std::move(c));
    if (child) *child = id;
    if (depth) *depth = d + 1;
    if (ntok) *ntok = tokens;
    return DH_OK;
}

dh_status dh_tree_append_token(dh_tree* t, uint64_t node, uint32_t token, uint32_t* cow_src,
                               uint32_t* cow_dst) {
    if (!t) return fail(DH_EINVAL, "tree is NULL");
    if (cow_src) *cow_src = DH_INVALID_PAGE;
    if (cow_dst) *cow_dst = DH_INVALID_PAGE;
    std::lock_guard<std::mutex> g(t->mu);
    auto it = t->nodes.find(node);
    if (it == t->nodes.end()) return fail(DH_EINVALID_NODE, "invalid node id: %llu", (unsigned long long)node);
    dh_block_table& tab = it->second.table;
    std::lock_guard<std::mutex> pg(t->pool->mu);
    if (needs_new_block(tab)) {
        uint32_t id;
        dh_status st = pool_allocate(t->pool, &id);
        if (st != DH_OK) return st;
        tab.blocks.push_back(id);
    }
    if (!tab.blocks.empty()) {
        const uint32_t last = tab.blocks.back();
        uint32_t nid;
        dh_status st = pool_cow(t->pool, last, &nid);
        if (st != DH_OK) return st;
        if (nid != last) {
            tab.blocks.back() = nid;
            if (cow_src) *cow_src = last;
            if (cow_dst) *cow_dst = nid;
        }
    }
    it->second.tokens.push_back(token);
    tab.num_tokens += 1;
    return DH_OK;
}

dh_status dh_tree_release(dh_tree* t, uint64_t node) {
    if (!t) return fail(DH_EINVAL, "tree is NULL");
    std::lock_guard<std::mutex> g(t->mu);
    auto it = t->nodes.find(node);
    if (it != t->nodes.end()) {
        it->second.active = false;
        if (it->second.parent != DH_INVALID_NODE) {
            auto p = t->nodes.find(it->second.parent);
            if (p != t->nodes.end() && p->second.num_children > 0) p->second.num_children--;
        }
    }
    // gc (state.rs:174-196): one pass over nodes that are inactive and childless.
    std::vector<uint64_t> victims;
    for (auto& kv : t->nodes)
        if (kv.first != DH_ROOT_NODE && !kv.second.active && kv.second.num_children == 0) victims.push_back(kv.first);
    std::lock_guard<std::mutex> pg(t->pool->mu);
    for (uint64_t id : victims) {
        auto n = t->nodes.find(id);
        for (uint32_t b : n->second.table.blocks) {
            if (b == DH_INVALID_PAGE) continue;
            dh_status st = pool_free(t->pool, b);
            if (st != DH_OK) return st;
        }
        t->nodes.erase(n);
    }
    return DH_OK;
}

dh_status dh_tree_get_node(const dh_tree* t, uint64_t node, dh_node_info* info) {
    if (!t || !info) return fail(DH_EINVAL, "NULL argument");
    std::lock_guard<std::mutex> g(t->mu);
    auto it = t->nodes.find(node);
    if (it == t->nodes.end()) return fail(DH_EINVALID_NODE, "invalid node id: %llu", (unsigned long long)node);
    info->id = it->second.id;
    info->parent = it->second.parent;
    info->num_tokens = it->second.table.num_tokens;
    info->num_children = it->second.num_children;
    info->is_active = it->second.active ? 1u : 0u;
    return DH_OK;
}

dh_status dh_tree_get_block_table(const dh_tree* t, uint64_t node, uint32_t* ids, uint32_t cap, uint32_t* n) {
    if (!t || !n) return fail(DH_EINVAL, "NULL argument");
    std::lock_guard<std::mutex> g(t->mu);
    auto it = t->nodes.find(node);
    if (it == t->nodes.end()) return fail(DH_EINVALID_NODE, "invalid node id: %llu", (unsigned long long)node);
    const auto& b = it->second.table.blocks;
    *n = uint32_t(b.size());
    for (uint32_t i = 0; i < b.size() && i < cap && ids; ++i) ids[i] = b[i];
    return DH_OK;
}

dh_status dh_tree_get_tokens(const dh_tree* t, uint64_t node, uint32_t* toks, uint32_t cap, uint32_t* n) {
    if (!t || !n) return fail(DH_EINVAL, "NULL argument");
    std::lock_guard<std::mutex> g(t->mu);
    auto it = t->nodes.find(node);
    if (it == t->nodes.end()) return fail(DH_EINVALID_NODE, "invalid node id: %llu", (unsigned long long)node);
    const auto& v = it->second.tokens;
    *n = uint32_t(v.size());
    for (uint32_t i = 0; i < v.size() && i < cap && toks; ++i) toks[i] = v[i];
    return DH_OK;
}

uint32_t dh_tree_num_nodes(const dh_tree* t) {
    if (!t) return 0;
    std::lock_guard<std::mutex> g(t->mu);
    return uint32_t(t->nodes.size());
}

uint32_t dh_tree_tokens_per_block(const dh_tree* t) { return t ? t->tokens_per_block : 0u; }

}  // extern "C"
