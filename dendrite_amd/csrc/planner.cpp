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

    // 3. Item classes and chunk sizes.  A segment with at most kWaveRows
    //    query rows becomes wave items (one wave each); a larger one becomes
    //    group items of up to in.group_rows rows whose four waves share every
    //    page through LDS.  Chunks split a segment's pages over items: more
    //    chunks give more parallelism and more partial states.
    auto is_group = [&](const Segment& sg) {
        return !in.wave_items_only && uint32_t(sg.seqs.size()) * r > uint32_t(kWaveRows);
    };
    uint32_t group_chunk = std::min<uint32_t>(in.shared_chunk_pages ? in.shared_chunk_pages : 32,
                                              kGroupMaxPages);
    // Wave items keep their page ids in registers (kWaveIdRegs x 64 at most).
    uint32_t wave_chunk = std::min<uint32_t>(in.private_chunk_pages ? in.private_chunk_pages : 8,
                                             uint32_t(kWaveIdRegs) * 64);
    const uint32_t target = in.target_items ? in.target_items : 1536;   // waves
    auto count_waves = [&](uint32_t gc, uint32_t wc) {
        uint64_t n = 0;
        for (const auto& sg : segs) {
            const uint32_t rows = uint32_t(sg.seqs.size()) * r;
            if (is_group(sg)) {
                n += uint64_t(ceil_div(uint32_t(sg.pages.size()), gc)) * ceil_div(rows, in.group_rows) *
                     in.hkv * kWaves;
            } else {
                n += uint64_t(ceil_div(uint32_t(sg.pages.size()), wc)) * ceil_div(rows, kWaveRows) * in.hkv;
            }
        }
        return n;
    };
    while (count_waves(group_chunk, wave_chunk) < target && (group_chunk > 8 || wave_chunk > 4)) {
        if (wave_chunk > 4) wave_chunk /= 2;
        if (count_waves(group_chunk, wave_chunk) >= target) break;
        if (group_chunk > 8) group_chunk /= 2;
    }
    // With default options and work to spare (four times the target), longer
    // chunks: fewer partial states for the merge to read and fewer item
    // starts.  Private chunks grow first (to 32 pages), then shared ones (to
    // kGroupMaxPages).  Measured on MI355X: C4 private 8 -> 32 pages took the
    // step from 322 to 250 us; C5 shared 32 -> 256 pages cut its merge from
    // 113 to 19 us.
    if (!in.shared_chunk_pages && !in.private_chunk_pages && !in.target_items) {
        constexpr uint32_t kMaxWaveChunk = 32;
        while (count_waves(group_chunk, wave_chunk) >= 4ull * target &&
               (wave_chunk < kMaxWaveChunk || group_chunk < uint32_t(kGroupMaxPages))) {
            if (wave_chunk < kMaxWaveChunk) wave_chunk *= 2;
            else group_chunk = std::min<uint32_t>(2 * group_chunk, kGroupMaxPages);
        }
    }

    // 4. Partial-state slots: one per (segment chunk, sequence), contiguous
    //    per sequence.
    std::vector<uint32_t> nchunks(segs.size());
    for (size_t s = 0; s < segs.size(); ++s) {
        const uint32_t ch = is_group(segs[s]) ? group_chunk : wave_chunk;
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

    // 5. Items.  Group items that read the same pages are kept together.
    std::vector<Group> groups;      // group items by (segment, chunk, head)
    std::vector<std::pair<double, Item>> waves;
    std::unordered_set<uint32_t> uniq;
    for (size_t s = 0; s < segs.size(); ++s) {
        const Segment& sg = segs[s];
        const bool grp = is_group(sg);
        const uint32_t np = uint32_t(sg.pages.size());
        const uint32_t base = uint32_t(out.pages.size());
        out.pages.insert(out.pages.end(), sg.pages.begin(), sg.pages.end());
        for (uint32_t p : sg.pages) uniq.insert(p);
        out.page_reads += np;
        const uint32_t nc = nchunks[s];
        const uint32_t rows = uint32_t(sg.seqs.size()) * r;
        const uint32_t block = grp ? in.group_rows : uint32_t(kWaveRows);
        const uint32_t nrb = ceil_div(rows, block);
        for (uint32_t ci = 0; ci < nc; ++ci) {
            const uint32_t p0 = uint32_t(uint64_t(ci) * np / nc);
            const uint32_t p1 = uint32_t(uint64_t(ci + 1) * np / nc);
            const uint32_t seq_off = uint32_t(out.seqslots.size());
            for (uint32_t b : sg.seqs) out.seqslots.push_back(SeqSlot{b, cursor[b]++});
            for (uint32_t h = 0; h < in.hkv; ++h) {
                Group gr;
                for (uint32_t rb = 0; rb < nrb; ++rb) {
                    Item it;
                    it.page_off = base + p0;
                    it.npages = p1 - p0;
                    it.seq_off = seq_off;
                    it.row_begin = rb * block;
                    it.nrows = std::min(block, rows - rb * block);
                    it.kv_head = h;
                    it.flags = (sg.tail && ci + 1 == nc) ? kItemTail : 0u;
                    it.tail_seq = sg.tail ? sg.seqs[0] : 0u;
                    const double cost = double(it.npages) * (2.0 + ceil_div(it.nrows, kTileRows));
                    if (grp) {
                        gr.items.push_back(it);
                        gr.cost += cost;
                    } else {
                        waves.emplace_back(cost, it);
                    }
                }
                if (grp) groups.push_back(std::move(gr));
            }
        }
    }
    out.unique_pages = uniq.size();

    // 6. Tasks.  Heaviest first.  Group tasks that read the same pages land
    //    on the same XCD (workgroups are dispatched round-robin over the 8
    //    XCDs, so task indices congruent mod 8 share an L2).  Wave items are
    //    packed four to a task, heaviest together.
    std::stable_sort(groups.begin(), groups.end(),
                     [](const Group& x, const Group& y) { return x.cost > y.cost; });
    std::stable_sort(waves.begin(), waves.end(),
                     [](const std::pair<double, Item>& x, const std::pair<double, Item>& y) {
                         return x.first > y.first;
                     });
    constexpr int kXcds = 8;
    std::vector<std::vector<Item>> q(kXcds);
    std::vector<double> qcost(kXcds, 0.0);
    for (auto& gr : groups) {
        int best = 0;
        for (int x = 1; x < kXcds; ++x)
            if (qcost[x] < qcost[best] || (qcost[x] == qcost[best] && q[x].size() < q[best].size()))
                best = x;
        for (auto& it : gr.items) q[best].push_back(it);
        qcost[best] += gr.cost;
    }
    std::vector<Item> gorder;
    size_t total = 0;
    for (auto& v : q) total += v.size();
    std::vector<size_t> pos(kXcds, 0);
    while (gorder.size() < total) {
        bool all = true;
        for (int x = 0; x < kXcds; ++x)
            if (pos[x] >= q[x].size()) all = false;
        if (all) {
            for (int x = 0; x < kXcds; ++x) gorder.push_back(q[x][pos[x]++]);
        } else {
            for (int x = 0; x < kXcds; ++x)
                while (pos[x] < q[x].size()) gorder.push_back(q[x][pos[x]++]);
        }
    }
    for (const Item& it : gorder) {
        out.tasks.push_back(Task{kTaskGroup, uint32_t(out.items.size()), 1u, 0u});
        out.items.push_back(it);
    }
    for (size_t i = 0; i < waves.size(); i += kWaves) {
        const uint32_t n = uint32_t(std::min<size_t>(kWaves, waves.size() - i));
        out.tasks.push_back(Task{kTaskWaves, uint32_t(out.items.size()), n, 0u});
        for (uint32_t k = 0; k < n; ++k) out.items.push_back(waves[i + k].second);
    }
    out.num_group_items = uint32_t(gorder.size());
    out.num_wave_items = uint32_t(waves.size());
    // The attention kernel derives a workgroup's items from its index alone
    // (AttendArgs): group task b runs item b, wave task b runs items
    // G + 4 (b - G) + w.  Check the emitted tasks against that mapping.
    for (size_t b = 0; b < out.tasks.size(); ++b) {
        const Task& t = out.tasks[b];
        const uint32_t G = out.num_group_items;
        const bool ok = b < G ? (t.kind == kTaskGroup && t.first == b && t.count == 1)
                              : (t.kind == kTaskWaves && t.first == G + kWaves * uint32_t(b - G) &&
                                 t.count == std::min<uint32_t>(kWaves, out.num_wave_items - kWaves * uint32_t(b - G)));
        if (!ok) {
            err = "internal: task " + std::to_string(b) + " does not follow the workgroup-to-item mapping";
            return DH_EINVAL;
        }
    }
    return DH_OK;
}

}  // namespace dh
