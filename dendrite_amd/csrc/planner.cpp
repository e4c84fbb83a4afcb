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

#include "dendrite_hip.h"

namespace dh {
namespace {

// A sequence's page list: a view of the caller's CSR indices, or of a copy
// with INVALID entries dropped.
struct PageList {
    const uint32_t* p = nullptr;
    uint32_t n = 0;
    size_t size() const { return n; }
    bool empty() const { return n == 0; }
    uint32_t operator[](size_t k) const { return p[k]; }
    uint32_t back() const { return p[n - 1]; }
    const uint32_t* data() const { return p; }
    const uint32_t* begin() const { return p; }
    const uint32_t* end() const { return p + n; }
};

// Compressed trie over block ids (a radix tree whose edges are runs of
// pages): a node is a run seq_pages[src][off .. off + len) that `count`
// sequences' page lists pass through.  Inserting a list compares whole runs
// and splits a node only where lists diverge or end, so once every list is
// in, the nodes reached by >= 2 lists are exactly the maximal runs shared
// by the same set of sequences: the shared segments.  A node's first child
// is kept inline; further children (forks) go to one map keyed by
// (node, first page).
struct RunNode {
    uint32_t src = 0, off = 0, len = 0;
    uint32_t count = 0;
    uint32_t segment = UINT32_MAX;
    uint32_t first_page = DH_INVALID_PAGE;   // first page of the inline child
    uint32_t first_child = 0;
    uint32_t nchildren = 0;
};

struct RunTrie {
    const std::vector<PageList>& lists;
    std::vector<RunNode> nodes;
    std::unordered_map<uint64_t, uint32_t> more;

    RunTrie(const std::vector<PageList>& l, size_t max_nodes) : lists(l) {
        nodes.reserve(max_nodes);
        nodes.emplace_back();   // root: the empty run
    }
    uint32_t page(const RunNode& n, uint32_t k) const { return lists[n.src][n.off + k]; }
    static uint64_t key(uint32_t node, uint32_t pg) { return (uint64_t(node) << 32) | pg; }

    uint32_t child(uint32_t cur, uint32_t pg) const {
        const RunNode& n = nodes[cur];
        if (n.nchildren && n.first_page == pg) return n.first_child;
        if (n.nchildren > 1) {
            const auto it = more.find(key(cur, pg));
            if (it != more.end()) return it->second;
        }
        return UINT32_MAX;
    }
    void set_child(uint32_t cur, uint32_t pg, uint32_t c, bool added) {
        RunNode& n = nodes[cur];
        if (n.nchildren == 0 || n.first_page == pg) {
            n.first_page = pg;
            n.first_child = c;
        } else {
            more[key(cur, pg)] = c;
        }
        if (added) n.nchildren++;
    }

    // Inserts the first n pages of sequence b's list.
    void insert(uint32_t b, size_t n) {
        const PageList& pl = lists[b];
        uint32_t cur = 0;
        size_t i = 0;
        while (i < n) {
            uint32_t c = child(cur, pl[i]);
            if (c == UINT32_MAX) {
                c = uint32_t(nodes.size());
                nodes.emplace_back();
                nodes[c].src = b;
                nodes[c].off = uint32_t(i);
                nodes[c].len = uint32_t(n - i);
                nodes[c].count = 1;
                set_child(cur, pl[i], c, true);
                return;
            }
            const uint32_t lim = uint32_t(std::min<size_t>(nodes[c].len, n - i));
            uint32_t m = 1;
            while (m < lim && page(nodes[c], m) == pl[i + m]) ++m;
            if (m < nodes[c].len) {   // split c: its first m pages become a new parent x
                const uint32_t x = uint32_t(nodes.size());
                nodes.emplace_back();
                RunNode& xn = nodes[x];
                RunNode& cn = nodes[c];
                xn.src = cn.src;
                xn.off = cn.off;
                xn.len = m;
                xn.count = cn.count;
                cn.off += m;
                cn.len -= m;
                xn.first_page = page(cn, 0);
                xn.first_child = c;
                xn.nchildren = 1;
                set_child(cur, pl[i], x, false);
                c = x;
            }
            nodes[c].count++;
            cur = c;
            i += m;
        }
    }

    // The nodes the first n pages of an inserted list pass through, in
    // order (after every insertion: a later split moves a node's front into
    // a new parent).
    void path(uint32_t b, size_t n, std::vector<uint32_t>& out) const {
        const PageList& pl = lists[b];
        uint32_t cur = 0;
        for (size_t i = 0; i < n;) {
            cur = child(cur, pl[i]);
            out.push_back(cur);
            i += nodes[cur].len;
        }
    }
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

// Wave chunk of a plan of wave items only that has work to spare: the
// candidate (from `cur` up to 128 pages) whose heaviest-first list schedule
// over the chip's wave slots (256 CUs x two workgroups x four waves) ends
// first.  An item costs its page pairs plus kStartPairs for its start (page
// ids, query, partial write).  Longer chunks mean fewer item starts and
// partial states, shorter ones a finer balance at the end of the step.  On
// MI355X, C4 (256 sequences of 32-256 FP8 pages): 32-page chunks 233 us a
// step, 64 226, 96 221 (chosen here), 128 235, 256 275.
uint32_t flat_wave_chunk(const std::vector<Segment>& segs, uint32_t r, uint32_t hkv, uint32_t cur) {
    constexpr uint32_t kSlots = 2048, kStartPairs = 3;
    std::vector<uint64_t> items;    // items of each cost (in pairs)
    std::vector<uint64_t> slots;    // slots at each load
    // Heaviest-first list scheduling, exact, in O(costs + loads): items of
    // one cost go to the least-loaded slots a level at a time, and the lowest
    // load only grows.  Loads stay below the mean plus the largest item.
    auto makespan = [&](uint32_t chunk) -> uint64_t {
        const uint32_t max_cost = kStartPairs + (chunk + 1) / 2;
        items.assign(max_cost + 1, 0);
        uint64_t total = 0;
        for (const auto& sg : segs) {
            const uint32_t np = uint32_t(sg.pages.size());
            const uint32_t nc = ceil_div(np, chunk);
            const uint64_t copies = uint64_t(ceil_div(uint32_t(sg.seqs.size()) * r, uint32_t(kWaveRows))) * hkv;
            for (uint32_t ci = 0; ci < nc; ++ci) {
                const uint32_t n = uint32_t(uint64_t(ci + 1) * np / nc - uint64_t(ci) * np / nc);
                const uint32_t c = kStartPairs + (n + 1) / 2;
                items[c] += copies;
                total += copies * c;
            }
        }
        const uint64_t cap = total / kSlots + max_cost + 1;
        if (cap > (uint64_t(1) << 26)) return 0;
        slots.assign(cap + 1, 0);
        slots[0] = kSlots;
        uint64_t lo = 0, end = 0;
        for (uint32_t c = max_cost; c >= 1; --c) {
            for (uint64_t k = items[c]; k != 0;) {
                while (slots[lo] == 0) ++lo;
                const uint64_t take = std::min(k, slots[lo]);
                slots[lo] -= take;
                slots[lo + c] += take;
                end = std::max(end, lo + c);
                k -= take;
            }
        }
        return end;
    };
    uint64_t best_t = makespan(cur);
    if (best_t == 0) return cur;
    uint32_t best = cur;
    for (uint32_t c : {48u, 64u, 96u, 128u}) {
        if (c <= cur || c > uint32_t(kWaveIdRegs) * 64) continue;
        const uint64_t t = makespan(c);
        if (t != 0 && t < best_t) {
            best_t = t;
            best = c;
        }
    }
    return best;
}

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
    //    skips blocks it has no KV for, attention/backend.rs:228-233): views
    //    of the indices, or of a filtered copy when there are INVALID ids.
    std::vector<PageList> seq_pages(B);
    std::vector<uint32_t> kept;
    bool any_invalid = false;
    for (uint32_t b = 0; b < B; ++b) {
        if (in.indptr[b + 1] < in.indptr[b]) {
            err = "indptr must be non-decreasing";
            return DH_EINVAL;
        }
        for (uint32_t k = in.indptr[b]; k < in.indptr[b + 1]; ++k) {
            const uint32_t p = in.indices[k];
            if (p == DH_INVALID_PAGE) {
                any_invalid = true;
                continue;
            }
            if (p >= in.num_pool_pages) {
                err = "page id " + std::to_string(p) + " outside the pool of " +
                      std::to_string(in.num_pool_pages) + " pages (sequence " +
                      std::to_string(b) + ")";
                return DH_EINVAL;
            }
        }
    }
    if (any_invalid) {
        kept.reserve(in.indptr[B]);
        for (uint32_t k = 0; k < in.indptr[B]; ++k)
            if (in.indices[k] != DH_INVALID_PAGE) kept.push_back(in.indices[k]);
    }
    for (uint32_t b = 0, o = 0; b < B; ++b) {
        if (any_invalid) {
            const uint32_t o0 = o;
            for (uint32_t k = in.indptr[b]; k < in.indptr[b + 1]; ++k) o += in.indices[k] != DH_INVALID_PAGE;
            seq_pages[b] = PageList{kept.data() + o0, o - o0};
        } else {
            seq_pages[b] = PageList{in.indices + in.indptr[b], in.indptr[b + 1] - in.indptr[b]};
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
        // Every list but its last page (only a sequence's last page may be
        // partial, so it stays private).  Each insertion adds at most two nodes.
        RunTrie trie(seq_pages, 2 * size_t(B) + 1);
        std::vector<std::vector<uint32_t>> paths(B);
        for (uint32_t b = 0; b < B; ++b)
            if (seq_pages[b].size() > 1) trie.insert(b, seq_pages[b].size() - 1);
        for (uint32_t b = 0; b < B; ++b)
            if (seq_pages[b].size() > 1) trie.path(b, seq_pages[b].size() - 1, paths[b]);
        // Shared nodes become segments in order of first use; a list's nodes
        // reached by it alone (all after its last shared one) and its last
        // page are its private pages.
        for (uint32_t b = 0; b < B; ++b) {
            for (const uint32_t u : paths[b]) {
                RunNode& n = trie.nodes[u];
                const uint32_t* run = seq_pages[n.src].data() + n.off;
                if (n.count < 2) {
                    private_pages[b].insert(private_pages[b].end(), run, run + n.len);
                    continue;
                }
                if (n.segment == UINT32_MAX) {
                    n.segment = uint32_t(segs.size());
                    segs.emplace_back();
                    segs.back().pages.assign(run, run + n.len);
                }
                seq_segs[b].push_back(n.segment);
                segs[n.segment].seqs.push_back(b);
            }
            if (!seq_pages[b].empty()) private_pages[b].push_back(seq_pages[b].back());
        }
        out.num_shared_segments = uint32_t(segs.size());
    } else {
        for (uint32_t b = 0; b < B; ++b) private_pages[b].assign(seq_pages[b].begin(), seq_pages[b].end());
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
    // A short segment of a few row blocks (at most 4 x 16 rows and 16 pages)
    // stays wave items: a group item's start (row targets, query rows and
    // first pairs, three dependent round trips) costs more than reading its
    // pages once per row block, mostly from L2.  C3 (whose level-1 nodes are
    // 8 pages under 64 rows), six rotations: 27.7 -> 26.8-27.5 us a step;
    // 16-page levels 42.0 -> 41.6 us.
    auto is_group = [&](const Segment& sg) {
        const uint32_t rows = uint32_t(sg.seqs.size()) * r;
        if (in.wave_items_only || rows <= uint32_t(kWaveRows)) return false;
        return rows > 4u * kWaveRows || sg.pages.size() > 16;
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
    // Below the target, chunks halve down to one page for wave items (C1,
    // one 32-page sequence: 4-page chunks 10.6 us a step, 1-page chunks 8.0)
    // and eight pages for group items.
    while (count_waves(group_chunk, wave_chunk) < target && (group_chunk > 8 || wave_chunk > 1)) {
        if (wave_chunk > 1) wave_chunk /= 2;
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
        bool any_group = false;
        for (const auto& sg : segs) any_group = any_group || is_group(sg);
        if (!any_group && wave_chunk >= kMaxWaveChunk)
            wave_chunk = flat_wave_chunk(segs, r, in.hkv, wave_chunk);
    }

    // 3b. Direct plans.  When no segment is shared and no item is a group
    //     item, each (sequence, KV head, row block) can be one workgroup: its
    //     pages in at most kWaves equal chunks, one per wave, whose partial
    //     states the workgroup merges itself, so the step is one launch.
    //     Taken when the chunks stay short (a sequence of at most
    //     kWaves * kDirectShortChunk pages: longer ones run faster as more,
    //     shorter chunks over more waves, merged by the merge kernel) or the
    //     workgroups alone give the target's worth of waves, each chunk fits
    //     a wave item's page ids, and every sequence has pages (the merge
    //     kernel writes the zeros of an empty one).
    bool direct = false;
    if (in.direct_ok && !segs.empty()) {
        constexpr uint32_t kDirectShortChunk = 4;
        bool ok = true;
        for (uint32_t b = 0; b < B; ++b) ok = ok && !seq_segs[b].empty();
        uint32_t max_np = 0;
        uint64_t blocks = 0;
        for (const auto& sg : segs) {
            ok = ok && sg.seqs.size() == 1 && !is_group(sg);
            max_np = std::max(max_np, uint32_t(sg.pages.size()));
            blocks += uint64_t(in.hkv) * ceil_div(r, uint32_t(kWaveRows));
        }
        ok = ok && ceil_div(max_np, uint32_t(kWaves)) <= uint32_t(kWaveIdRegs) * 64 &&
             (max_np <= kWaves * kDirectShortChunk || blocks * kWaves >= target);
        direct = ok;
    }
    out.direct = direct;

    // 4. Partial-state slots: one per (segment chunk, sequence), contiguous
    //    per sequence.
    std::vector<uint32_t> nchunks(segs.size());
    for (size_t s = 0; s < segs.size(); ++s) {
        const uint32_t ch = is_group(segs[s]) ? group_chunk : wave_chunk;
        nchunks[s] = direct ? std::min<uint32_t>(kWaves, uint32_t(segs[s].pages.size()))
                            : ceil_div(uint32_t(segs[s].pages.size()), ch);
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
    out.tail_off.assign(B, 0);
    out.tail_n.assign(B, 0);
    out.tail_cap.assign(B, 0);
    std::vector<std::pair<double, Item>> waves;
    std::vector<std::pair<double, std::vector<Item>>> direct_tasks;
    // Distinct pages of the plan, for the statistics: a bitmap over the pool.
    std::vector<uint64_t> seen((uint64_t(in.num_pool_pages) + 63) / 64, 0);
    uint64_t uniq = 0;
    for (size_t s = 0; s < segs.size(); ++s) {
        const Segment& sg = segs[s];
        const bool grp = is_group(sg);
        const uint32_t np = uint32_t(sg.pages.size());
        const uint32_t base = uint32_t(out.pages.size());
        out.pages.insert(out.pages.end(), sg.pages.begin(), sg.pages.end());
        if (sg.tail) {
            // Room for the sequence's last chunk to grow in place.
            const uint32_t b = sg.seqs[0];
            const uint32_t p0 = uint32_t(uint64_t(nchunks[s] - 1) * sg.pages.size() / nchunks[s]);
            out.tail_off[b] = base + p0;
            out.tail_n[b] = uint32_t(sg.pages.size()) - p0;
            out.tail_cap[b] = std::max(out.tail_n[b], std::min<uint32_t>(out.tail_n[b] + kTailSlack, kMaxItemPages));
            out.pages.insert(out.pages.end(), out.tail_cap[b] - out.tail_n[b], DH_INVALID_PAGE);
        }
        for (uint32_t p : sg.pages) {
            const uint64_t bit = 1ull << (p & 63);
            uniq += (seen[p >> 6] & bit) == 0;
            seen[p >> 6] |= bit;
        }
        out.page_reads += np;
        const uint32_t nc = nchunks[s];
        const uint32_t rows = uint32_t(sg.seqs.size()) * r;
        const uint32_t block = grp ? in.group_rows : uint32_t(kWaveRows);
        const uint32_t nrb = ceil_div(rows, block);
        if (direct) {
            // One task per (KV head, row block): its chunks, then empty
            // items up to kWaves (kept in this order by the task packing).
            const uint32_t seq_off = uint32_t(out.seqslots.size());
            const uint32_t b = sg.seqs[0];
            for (uint32_t ci = 0; ci < nc; ++ci) out.seqslots.push_back(SeqSlot{b, cursor[b]++});
            for (uint32_t h = 0; h < in.hkv; ++h) {
                for (uint32_t rb = 0; rb < nrb; ++rb) {
                    double cost = 0.0;
                    std::vector<Item> task;
                    for (uint32_t ci = 0; ci < uint32_t(kWaves); ++ci) {
                        Item it;
                        const uint32_t p0 = ci < nc ? uint32_t(uint64_t(ci) * np / nc) : np;
                        const uint32_t p1 = ci < nc ? uint32_t(uint64_t(ci + 1) * np / nc) : np;
                        it.page_off = base + (ci < nc ? p0 : 0u);
                        it.npages = p1 - p0;
                        it.seq_off = seq_off + (ci < nc ? ci : 0u);
                        it.row_begin = rb * block;
                        it.nrows = std::min(block, rows - rb * block);
                        it.kv_head = h;
                        it.flags = (sg.tail && ci + 1 == nc) ? kItemTail : 0u;
                        it.tail_seq = sg.tail ? b : 0u;
                        cost += double(it.npages);
                        task.push_back(it);
                    }
                    direct_tasks.emplace_back(cost, std::move(task));
                }
            }
            continue;
        }
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
    out.unique_pages = uniq;

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
    // Direct tasks, heaviest first; each keeps its kWaves items in order.
    std::stable_sort(direct_tasks.begin(), direct_tasks.end(),
                     [](const auto& x, const auto& y) { return x.first > y.first; });
    for (const auto& dt : direct_tasks) {
        out.tasks.push_back(Task{kTaskWaves, uint32_t(out.items.size()), uint32_t(kWaves), 0u});
        for (const Item& it : dt.second) out.items.push_back(it);
    }
    out.num_group_items = uint32_t(gorder.size());
    out.num_wave_items = uint32_t(waves.size() + direct_tasks.size() * kWaves);
    for (size_t i = 0; i < out.items.size(); ++i)
        if (out.items[i].npages > (i < out.num_group_items ? uint32_t(kGroupMaxPages) : kMaxItemPages)) {
            err = "internal: an item of " + std::to_string(out.items[i].npages) + " pages";
            return DH_EINVAL;
        }
    // The items of each sequence's last chunk, by final item index.
    out.tail_item_ptr.assign(B + 1, 0);
    for (const Item& it : out.items)
        if (it.flags & kItemTail) out.tail_item_ptr[it.tail_seq + 1]++;
    for (uint32_t b = 0; b < B; ++b) out.tail_item_ptr[b + 1] += out.tail_item_ptr[b];
    out.tail_items.resize(out.tail_item_ptr[B]);
    {
        std::vector<uint32_t> fill(out.tail_item_ptr.begin(), out.tail_item_ptr.end() - 1);
        for (uint32_t i = 0; i < uint32_t(out.items.size()); ++i)
            if (out.items[i].flags & kItemTail) out.tail_items[fill[out.items[i].tail_seq]++] = i;
    }
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

// Prefill items: for each sequence, KV head and block of query tokens
// (group_rows / r tokens, their r heads each a row), the KV pages the block's
// last query sees, cut into chunks of chunk_pages.  Chunk starts stay below
// the block's first query's token count (the last chunk absorbs the rest,
// the diagonal included), so every row sees at least one token of every
// item it is in.  Items: heaviest first; one workgroup each.
int build_prefill_plan(const PrefillInput& in, HostPlan& out, std::string& err) {
    out = HostPlan();
    const uint32_t B = in.batch;
    if (in.hkv == 0 || in.hq % in.hkv != 0) {
        err = "num_heads must be divisible by num_kv_heads";
        return DH_EINVAL;
    }
    const uint32_t r = in.hq / in.hkv;
    if (r > in.group_rows) {
        err = "more query heads per KV head than rows in a work item";
        return DH_EUNSUPPORTED;
    }
    const uint32_t tpb = in.group_rows / r;   // query tokens per block
    // Page lists (INVALID dropped) and the virtual sequences.
    std::vector<std::vector<uint32_t>> pl(B);
    std::vector<uint32_t> q_off(B + 1, 0);
    for (uint32_t b = 0; b < B; ++b) {
        if (in.indptr[b + 1] < in.indptr[b]) {
            err = "indptr must be non-decreasing";
            return DH_EINVAL;
        }
        for (uint32_t k = in.indptr[b]; k < in.indptr[b + 1]; ++k) {
            const uint32_t p = in.indices[k];
            if (p == DH_INVALID_PAGE) continue;
            if (p >= in.num_pool_pages) {
                err = "page id " + std::to_string(p) + " outside the pool (sequence " + std::to_string(b) + ")";
                return DH_EINVAL;
            }
            pl[b].push_back(p);
        }
        const uint64_t np = pl[b].size(), kv = in.kv_len[b], q = in.q_len[b];
        if (kv > np * kPageSize || (np && kv <= (np - 1) * kPageSize) || (!np && kv)) {
            err = "sequence " + std::to_string(b) + ": " + std::to_string(kv) + " tokens do not fill its " +
                  std::to_string(np) + " pages (the last one holds 1..16)";
            return DH_EINVAL;
        }
        if (q > kv) {
            err = "sequence " + std::to_string(b) + ": more queries than tokens";
            return DH_EINVAL;
        }
        if (kv > DH_MAX_SEQ_LEN) {
            err = "sequence " + std::to_string(b) + " exceeds MAX_SEQ_LEN";
            return DH_EINVAL;
        }
        q_off[b + 1] = q_off[b] + uint32_t(q);
        out.total_pages += np;
    }
    const uint32_t nq = q_off[B];
    out.row_len.resize(nq);
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t i = 0; i < in.q_len[b]; ++i)
            out.row_len[q_off[b] + i] = in.causal ? in.kv_len[b] - in.q_len[b] + i + 1 : in.kv_len[b];
    auto len_of = [&](uint32_t b, uint32_t i) { return out.row_len[q_off[b] + i]; };

    // Chunk size: one chunk per block when blocks alone fill the chip, at
    // most kPrefillMaxChunk pages: an item's page ids are staged in an LDS
    // list of kPrefillMaxPages entries, and the last chunk of a block also
    // takes the pages between its first and last query (at most
    // tpb / 16 + 1 more).
    const uint32_t kPrefillMaxChunk = uint32_t(kPrefillMaxPages) - (tpb + kPageSize - 1) / kPageSize - 1;
    uint64_t n_blocks = 0;
    for (uint32_t b = 0; b < B; ++b) n_blocks += (in.q_len[b] + tpb - 1) / tpb;
    uint32_t chunk = in.chunk_pages;
    if (!chunk && n_blocks * in.hkv >= 512) {
        chunk = UINT32_MAX;
    } else if (!chunk) {
        // Fewer blocks than the chip holds: cut their pages into about 1024
        // items (four per CU), at least 32 pages each.
        uint64_t seen = 0;   // pages the blocks' last queries see
        for (uint32_t b = 0; b < B; ++b)
            for (uint32_t i0 = 0; i0 < in.q_len[b]; i0 += tpb)
                seen += (len_of(b, std::min(in.q_len[b], i0 + tpb) - 1) + kPageSize - 1) / kPageSize;
        chunk = uint32_t(std::max<uint64_t>(32, (seen * in.hkv + 1023) / 1024));
    }
    chunk = std::min(chunk, kPrefillMaxChunk);

    // Blocks and their chunks: (sequence, token range, page range).
    struct Piece {
        uint32_t b, i0, i1, p0, p1;
    };
    std::vector<Piece> pieces;
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t i0 = 0; i0 < in.q_len[b]; i0 += tpb) {
            const uint32_t i1 = std::min(in.q_len[b], i0 + tpb);
            const uint32_t lmin = len_of(b, i0), lmax = len_of(b, i1 - 1);
            const uint32_t pend = (lmax + kPageSize - 1) / kPageSize;
            const uint32_t plast = (lmin - 1) / kPageSize;       // a chunk may start at or below this page
            uint32_t p0 = 0;
            while (true) {
                const uint64_t nx = uint64_t(p0) + chunk;
                if (nx > plast || nx >= pend) {
                    pieces.push_back(Piece{b, i0, i1, p0, pend});
                    break;
                }
                pieces.push_back(Piece{b, i0, i1, p0, uint32_t(nx)});
                p0 = uint32_t(nx);
            }
        }
    }
    for (const Piece& pc : pieces)
        if (pc.p1 - pc.p0 > uint32_t(kPrefillMaxPages)) {
            err = "internal: a prefill item of " + std::to_string(pc.p1 - pc.p0) + " pages";
            return DH_EINVAL;
        }
    // Partial slots: one per (chunk, query), contiguous per query.
    std::vector<uint32_t> count(nq, 0);
    for (const Piece& pc : pieces)
        for (uint32_t i = pc.i0; i < pc.i1; ++i) count[q_off[pc.b] + i]++;
    out.slot_ptr.assign(nq + 1, 0);
    for (uint32_t v = 0; v < nq; ++v) out.slot_ptr[v + 1] = out.slot_ptr[v] + count[v];
    out.num_slots = out.slot_ptr[nq];
    std::vector<uint32_t> cursor(out.slot_ptr.begin(), out.slot_ptr.end() - 1);
    // Page lists into the plan, one copy per sequence.
    std::vector<uint32_t> page_base(B);
    for (uint32_t b = 0; b < B; ++b) {
        page_base[b] = uint32_t(out.pages.size());
        out.pages.insert(out.pages.end(), pl[b].begin(), pl[b].end());
    }
    struct Cand {
        double cost;
        Item it;
        ItemLim lim;
    };
    std::vector<Cand> cands;
    for (const Piece& pc : pieces) {
        const uint32_t seq_off = uint32_t(out.seqslots.size());
        for (uint32_t i = pc.i0; i < pc.i1; ++i) {
            const uint32_t v = q_off[pc.b] + i;
            out.seqslots.push_back(SeqSlot{v, cursor[v]++});
        }
        const uint32_t tok0 = pc.p0 * kPageSize, tok_end = std::min(pc.p1 * kPageSize, in.kv_len[pc.b]);
        ItemLim lim;
        lim.tok0 = tok0;
        lim.lmin = std::min(len_of(pc.b, pc.i0), tok_end);
        lim.lmax = std::min(len_of(pc.b, pc.i1 - 1), tok_end);
        lim.pad = 0;
        for (uint32_t h = 0; h < in.hkv; ++h) {
            Item it;
            it.page_off = page_base[pc.b] + pc.p0;
            it.npages = pc.p1 - pc.p0;
            it.seq_off = seq_off;
            it.row_begin = 0;
            it.nrows = (pc.i1 - pc.i0) * r;
            it.kv_head = h;
            it.flags = kItemCausal;
            it.tail_seq = 0;
            const double cost = double(it.npages) * (2.0 + (it.nrows + kTileRows - 1) / kTileRows);
            cands.push_back(Cand{cost, it, lim});
        }
        out.page_reads += uint64_t(pc.p1 - pc.p0);
    }
    std::stable_sort(cands.begin(), cands.end(), [](const Cand& x, const Cand& y) { return x.cost > y.cost; });
    for (const Cand& c : cands) {
        out.tasks.push_back(Task{kTaskGroup, uint32_t(out.items.size()), 1u, 0u});
        out.items.push_back(c.it);
        out.item_lim.push_back(c.lim);
    }
    out.num_group_items = uint32_t(out.items.size());
    out.num_wave_items = 0;
    out.num_segments = uint32_t(pieces.size());
    out.num_shared_segments = 0;
    uint64_t uniq = 0;
    for (uint32_t b = 0; b < B; ++b) uniq += pl[b].size();
    out.unique_pages = uniq;
    return DH_OK;
}

}  // namespace dh
