// Cascade planner: finds the runs of pages that several sequences share
// (the copy-on-write prefixes TreeState::fork creates by cloning a block
// table and bumping every block's refcount, crates/dendrite-core/src/tree/
// state.rs:49-84, node.rs:72-81) so a decode step reads each shared page once
// for all the sequences that reference it, then cuts the step into work items.
//
// The trie is keyed by physical page id, the radix-tree idea of
// crates/dendrite-core/src/cache/radix.rs applied to block ids instead of
// tokens.  Each sequence's last page stays private: only it may be partial
// (its length is a per-call input), and sequences that end on the same page
// are rare.
#include "planner.hpp"

#include <algorithm>
#include <unordered_map>
#include <unordered_set>

#include "dendrite_hip.h"

namespace dh {
namespace {

struct TrieNode {
    uint32_t page;
    uint32_t count = 0;                 // sequences whose path passes here
    uint32_t segment = UINT32_MAX;      // shared segment id (count >= 2)
    std::unordered_map<uint32_t, uint32_t> children;
};

struct Segment {
    std::vector<uint32_t> pages;
    std::vector<uint32_t> seqs;
    bool tail = false;
};

struct Group {                          // items that read the same pages
    std::vector<Item> items;
    double cost = 0.0;
};

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

}  // namespace

int build_plan(const PlanInput& in, HostPlan& out, std::string& err) {
    out = HostPlan();
    const uint32_t B = in.batch;
    if (in.hkv == 0 || in.hq % in.hkv != 0) {
        err = "num_heads must be divisible by num_kv_heads";
        return DH_EINVAL;
    }
    const uint32_t r = in.hq / in.hkv;
    const uint32_t rpi = in.rows_per_item;

    // 1. Page lists with INVALID entries dropped (ReferenceBackend::decode
    //    skips blocks it has no KV for, attention/backend.rs:228-233).
    std::vector<std::vector<uint32_t>> seq_pages(B);
    for (uint32_t b = 0; b < B; ++b) {
        if (in.indptr[b + 1] < in.indptr[b]) {
            err = "indptr must be non-decreasing";
            return DH_EINVAL;
        }
        for (uint32_t k = in.indptr[b]; k < in.indptr[b + 1]; ++k) {
            const uint32_t p = in.indices[k];
            if (p == DH_INVALID_PAGE) continue;
            if (p >= in.num_pool_pages) {
                err = "page id " + std::to_string(p) + " outside the pool of " +
                      std::to_string(in.num_pool_pages) + " pages (sequence " +
                      std::to_string(b) + ")";
                return DH_EINVAL;
            }
            seq_pages[b].push_back(p);
        }
        if (uint64_t(seq_pages[b].size()) * kPageSize > DH_MAX_SEQ_LEN) {
            err = "sequence " + std::to_string(b) + " exceeds MAX_SEQ_LEN";
            return DH_EINVAL;
        }
        out.total_pages += seq_pages[b].size();
    }

    // 2. Segments.
    std::vector<Segment> segs;
    std::vector<std::vector<uint32_t>> seq_segs(B);   // segment ids per sequence
    std::vector<std::vector<uint32_t>> private_pages(B);
    if (in.cascade) {
        std::vector<TrieNode> nodes(1);
        nodes[0].page = DH_INVALID_PAGE;
        std::vector<std::vector<uint32_t>> paths(B);
        for (uint32_t b = 0; b < B; ++b) {
            const auto& pl = seq_pages[b];
            uint32_t cur = 0;
            for (size_t k = 0; k + 1 < pl.size(); ++k) {
                auto it = nodes[cur].children.find(pl[k]);
                uint32_t nxt;
                if (it == nodes[cur].children.end()) {
                    nxt = uint32_t(nodes.size());
                    nodes[cur].children.emplace(pl[k], nxt);
                    nodes.emplace_back();
                    nodes.back().page = pl[k];
                } else {
                    nxt = it->second;
                }
                nodes[nxt].count++;
                paths[b].push_back(nxt);
                cur = nxt;
            }
        }
        // A shared segment is a maximal chain of nodes with count >= 2 where
        // each node is the only child of the previous one and keeps its count
        // (so the chain is referenced by exactly the same sequences).
        for (uint32_t b = 0; b < B; ++b) {
            const auto& path = paths[b];
            uint32_t prev = 0;
            for (size_t k = 0; k < path.size(); ++k) {
                const uint32_t u = path[k];
                TrieNode& n = nodes[u];
                if (n.count < 2) {
                    private_pages[b].push_back(n.page);
                } else {
                    if (n.segment == UINT32_MAX) {
                        const bool extend = prev != 0 && nodes[prev].count == n.count &&
                                            nodes[prev].children.size() == 1 &&
                                            nodes[prev].segment != UINT32_MAX;
                        if (extend) {
                            n.segment = nodes[prev].segment;
                            segs[n.segment].pages.push_back(n.page);
                        } else {
                            n.segment = uint32_t(segs.size());
                            segs.emplace_back();
                            segs.back().pages.push_back(n.page);
                        }
                    }
                    if (seq_segs[b].empty() || seq_segs[b].back() != n.segment) {
                        seq_segs[b].push_back(n.segment);
                        segs[n.segment].seqs.push_back(b);
                    }
                }
                prev = u;
            }
            if (!seq_pages[b].empty()) private_pages[b].push_back(seq_pages[b].back());
        }
        out.num_shared_segments = uint32_t(segs.size());
    } else {
        for (uint32_t b = 0; b < B; ++b) private_pages[b] = seq_pages[b];
    }
    for (uint32_t b = 0; b < B; ++b) {
        if (private_pages[b].empty()) continue;
        seq_segs[b].push_back(uint32_t(segs.size()));
        segs.emplace_back();
        segs.back().pages = private_pages[b];
        segs.back().seqs.push_back(b);
        segs.back().tail = true;
    }
    out.num_segments = uint32_t(segs.size());

    // 3. Chunk sizes.  A chunk is the page run of one item; its four waves
    //    split it.  More chunks mean more parallelism and more partial states.
    uint32_t shared_chunk = in.shared_chunk_pages ? in.shared_chunk_pages : 64;
    uint32_t private_chunk = in.private_chunk_pages ? in.private_chunk_pages : 64;
    const uint32_t target = in.target_items ? in.target_items : 1024;
    auto count_items = [&](uint32_t sc, uint32_t pc) {
        uint64_t n = 0;
        for (const auto& s : segs) {
            const uint32_t ch = s.tail ? pc : sc;
            const uint32_t rows = uint32_t(s.seqs.size()) * r;
            n += uint64_t(ceil_div(uint32_t(s.pages.size()), ch)) * ceil_div(rows, rpi) * in.hkv;
        }
        return n;
    };
    while (count_items(shared_chunk, private_chunk) < target && (shared_chunk > 8 || private_chunk > 8)) {
        if (shared_chunk > 8) shared_chunk /= 2;
        if (private_chunk > 8) private_chunk /= 2;
    }

    // 4. Partial-state slots: one per (segment chunk, sequence), contiguous
    //    per sequence.
    std::vector<uint32_t> nchunks(segs.size());
    for (size_t s = 0; s < segs.size(); ++s) {
        const uint32_t ch = segs[s].tail ? private_chunk : shared_chunk;
        nchunks[s] = ceil_div(uint32_t(segs[s].pages.size()), ch);
    }
    out.slot_ptr.assign(B + 1, 0);
    for (uint32_t b = 0; b < B; ++b) {
        uint32_t n = 0;
        for (uint32_t s : seq_segs[b]) n += nchunks[s];
        out.slot_ptr[b + 1] = out.slot_ptr[b] + n;
    }
    out.num_slots = out.slot_ptr[B];
    std::vector<uint32_t> cursor(out.slot_ptr.begin(), out.slot_ptr.end() - 1);

    // 5. Items, grouped by the pages they read.
    std::vector<Group> groups;
    std::unordered_set<uint32_t> uniq;
    for (size_t s = 0; s < segs.size(); ++s) {
        const Segment& sg = segs[s];
        const uint32_t np = uint32_t(sg.pages.size());
        const uint32_t base = uint32_t(out.pages.size());
        out.pages.insert(out.pages.end(), sg.pages.begin(), sg.pages.end());
        for (uint32_t p : sg.pages) uniq.insert(p);
        out.page_reads += np;
        const uint32_t nc = nchunks[s];
        const uint32_t rows = uint32_t(sg.seqs.size()) * r;
        const uint32_t nrb = ceil_div(rows, rpi);
        for (uint32_t ci = 0; ci < nc; ++ci) {
            const uint32_t p0 = uint32_t(uint64_t(ci) * np / nc);
            const uint32_t p1 = uint32_t(uint64_t(ci + 1) * np / nc);
            const uint32_t seq_off = uint32_t(out.seqslots.size());
            for (uint32_t b : sg.seqs) out.seqslots.push_back(SeqSlot{b, cursor[b]++});
            for (uint32_t h = 0; h < in.hkv; ++h) {
                Group grp;
                for (uint32_t rb = 0; rb < nrb; ++rb) {
                    Item it;
                    it.page_off = base + p0;
                    it.npages = p1 - p0;
                    it.seq_off = seq_off;
                    it.row_begin = rb * rpi;
                    it.nrows = std::min(rpi, rows - rb * rpi);
                    it.kv_head = h;
                    const bool last = sg.tail && ci + 1 == nc;
                    it.flags = last ? kItemTail : 0u;
                    it.tail_seq = sg.tail ? sg.seqs[0] : 0u;
                    grp.cost += double(it.npages) * (2.0 + ceil_div(it.nrows, 16));
                    grp.items.push_back(it);
                }
                groups.push_back(std::move(grp));
            }
        }
    }
    out.unique_pages = uniq.size();

    // 6. Order: heaviest groups first; the items of one group land on the
    //    same XCD (workgroups are dispatched round-robin over the 8 XCDs, so
    //    indices congruent mod 8 share an L2) to reuse the group's pages in L2.
    std::stable_sort(groups.begin(), groups.end(),
                     [](const Group& a, const Group& b) { return a.cost > b.cost; });
    constexpr int kXcds = 8;
    std::vector<std::vector<Item>> q(kXcds);
    std::vector<double> qcost(kXcds, 0.0);
    for (auto& grp : groups) {
        int best = 0;
        for (int x = 1; x < kXcds; ++x)
            if (qcost[x] < qcost[best] ||
                (qcost[x] == qcost[best] && q[x].size() < q[best].size()))
                best = x;
        for (auto& it : grp.items) q[best].push_back(it);
        qcost[best] += grp.cost;
    }
    size_t total = 0;
    for (auto& v : q) total += v.size();
    out.items.reserve(total);
    std::vector<size_t> pos(kXcds, 0);
    while (out.items.size() < total) {
        bool all = true;
        for (int x = 0; x < kXcds; ++x)
            if (pos[x] >= q[x].size()) all = false;
        if (all) {
            for (int x = 0; x < kXcds; ++x) out.items.push_back(q[x][pos[x]++]);
        } else {
            for (int x = 0; x < kXcds; ++x)
                while (pos[x] < q[x].size()) out.items.push_back(q[x][pos[x]++]);
        }
    }
    return DH_OK;
}

}  // namespace dh
