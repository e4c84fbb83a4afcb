"""Host planner (dh_plan_inspect, CPU only): every query row attends every
page of its sequence exactly once, partial-state slots are written once, and
with the cascade plan every page of a tree is read once per KV head.

What the reference fixes here: the pages a sequence attends are its block
table's entries in order minus INVALID ids (ReferenceBackend::decode,
attention/backend.rs:228-233); ids beyond the pool and bad head shapes are
rejected the way BatchDecodeKernel::new rejects them (dendrite-ffi/src/
flashinfer/batch_decode.rs:33-45).
"""
from collections import Counter

import numpy as np
import pytest

from dendrite_amd import DhError, _lib, workloads
from dendrite_amd.backend import AttentionConfig, plan_inspect

INVALID = _lib.INVALID_PAGE


def _cfg(w):
    c = AttentionConfig(w.hq, w.hkv, w.d)
    c.q_dtype, c.kv_format, c.gqa_mapping = w.q_dtype, w.kv_format, w.gqa_mapping
    return c


def _check_cover(w, plan):
    hq, hkv = w.hq, w.hkv
    r = hq // hkv
    B = w.batch
    seqslots = plan["seqslots"]
    pages = plan["pages"]
    got = {}                       # (b, kv head, j) -> Counter of pages
    written = Counter()            # (slot, kv head, j)
    slot_owner = {}
    items = plan["items"]
    for k, it in enumerate(items):
        pl = pages[it["page_off"]:it["page_off"] + it["npages"]]
        if it["npages"] == 0:
            # Only direct plans pad a workgroup's four wave items with empty
            # ones, after the chunks, rows equal to the task's first item.
            assert plan["stats"]["direct"] == 1
            first = items[k - k % 4]
            assert first["npages"] >= 1 and (it["row_begin"], it["nrows"], it["kv_head"]) == \
                (first["row_begin"], first["nrows"], first["kv_head"])
            continue
        for rho in range(it["row_begin"], it["row_begin"] + it["nrows"]):
            b, slot = (int(x) for x in seqslots[it["seq_off"] + rho // r])
            j = rho % r
            got.setdefault((b, it["kv_head"], j), Counter()).update(int(p) for p in pl)
            written[(slot, it["kv_head"], j)] += 1
            assert slot_owner.setdefault(slot, b) == b, "a slot serves two sequences"
    for b in range(B):
        want = Counter(int(p) for p in w.indices[w.indptr[b]:w.indptr[b + 1]] if p != INVALID)
        for h in range(hkv):
            for j in range(r):
                assert got.get((b, h, j), Counter()) == want, f"sequence {b} head {h} row {j}"
    assert all(v == 1 for v in written.values()), "a partial state is written twice"
    assert len(slot_owner) == plan["stats"]["num_partials"]
    return got


CASES = {
    "c1": workloads.c1(),
    "c2": workloads.c2(),
    "c3_small": workloads.c3(root_pages=40, levels=2, level_pages=3, pool_pages=4096),
    "c4_small": workloads.c4(n_seqs=24, tmin=40, tmax=700, pool_pages=4096),
    "c5_small": workloads.c5(requests=2, prefix_pages=40, beams=4, suffix_pages=5, pool_pages=2048),
    "random_bf16": workloads.random_tree(11, 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, n_leaves=10,
                                         pool_pages=512),
    "random_f32": workloads.random_tree(12, 32, 4, 64, _lib.DTYPE_F32, _lib.KV_F32, n_leaves=10,
                                        pool_pages=512),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("cascade", [True, False])
def test_every_row_reads_its_pages_once(name, cascade):
    w = CASES[name]
    plan = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices, cascade=cascade)
    _check_cover(w, plan)
    st = plan["stats"]
    assert st["total_pages"] == sum(1 for p in w.indices if p != INVALID)
    if not cascade:
        assert st["page_reads"] == st["total_pages"]


@pytest.mark.parametrize("opts", [dict(shared_chunk_pages=8), dict(private_chunk_pages=2),
                                  dict(target_items=20000), dict(target_items=1)])
def test_chunking_options_keep_coverage(opts):
    w = CASES["c3_small"]
    _check_cover(w, plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices, **opts))


def test_c3_tree_reads_each_page_once_per_head():
    w = workloads.c3()
    plan = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices)
    st = plan["stats"]
    assert st["unique_pages"] == 1184 and st["page_reads"] == 1184
    assert st["total_pages"] == 64 * 536
    # every page id appears once in the plan's page list (per KV head the
    # items of a chunk share that list); the INVALID entries are the room
    # reserved after each sequence's last chunk
    ids = plan["pages"][plan["pages"] != INVALID]
    assert len(ids) == 1184 and Counter(ids.tolist()).most_common(1)[0][1] == 1


@pytest.mark.parametrize("name", ["c3_small", "c4_small", "c5_small"])
def test_last_chunks_have_room_to_grow(name):
    """Each sequence's last chunk is followed by 16 reserved (INVALID)
    entries of the page list, which dh_plan_update fills in place; no other
    item's pages reach into them."""
    w = CASES[name]
    plan = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices)
    pages = plan["pages"]
    reserved = set()
    tails = set()
    for it in plan["items"]:
        if it["flags"] & 1:
            end = it["page_off"] + it["npages"]
            assert np.all(pages[end:end + 16] == INVALID), "no room after a last chunk"
            reserved.update(range(end, end + 16))
            tails.add(it["tail_seq"])
    assert tails == set(range(w.batch))
    for it in plan["items"]:
        span = set(range(it["page_off"], it["page_off"] + it["npages"]))
        assert not span & reserved
    assert np.count_nonzero(pages == INVALID) == 16 * w.batch


def test_tail_items_name_their_sequence():
    w = CASES["c4_small"]
    plan = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices)
    tails = {}
    for it in plan["items"]:
        if it["flags"] & 1:
            last = int(plan["pages"][it["page_off"] + it["npages"] - 1])
            tails.setdefault(it["tail_seq"], set()).add(last)
    for b in range(w.batch):
        tbl = [p for p in w.indices[w.indptr[b]:w.indptr[b + 1]] if p != INVALID]
        assert tails[b] == {tbl[-1]}


def test_invalid_ids_and_empty_tables():
    w = workloads.custom([[3, INVALID, 5], [], [INVALID], [3, INVALID, 5, 9]], 8, 2, 64,
                         _lib.DTYPE_BF16, _lib.KV_BF16, 16)
    plan = plan_inspect(_cfg(w), 16, w.indptr, w.indices)
    _check_cover(w, plan)


def _err(fn):
    with pytest.raises(DhError) as e:
        fn()
    return e.value.status


def test_rejects_bad_inputs():
    w = CASES["c2"]
    cfg = _cfg(w)
    assert _err(lambda: plan_inspect(cfg, 16, w.indptr, w.indices)) == _lib.DH_EINVAL   # id >= pool
    bad = AttentionConfig(32, 4, 96)
    assert _err(lambda: plan_inspect(bad, w.num_pool_pages, w.indptr, w.indices)) == _lib.DH_EINVAL
    bad = AttentionConfig(30, 4, 64)
    assert _err(lambda: plan_inspect(bad, w.num_pool_pages, w.indptr, w.indices)) == _lib.DH_EINVAL
    # sliding_window is accepted and ignored, like every Dendrite backend
    sw = _cfg(w).with_sliding_window(128)
    a = plan_inspect(sw, w.num_pool_pages, w.indptr, w.indices)
    assert a["stats"] == plan_inspect(cfg, w.num_pool_pages, w.indptr, w.indices)["stats"]
    ip = np.array([0, 3, 2], dtype=np.uint32)
    assert _err(lambda: plan_inspect(cfg, w.num_pool_pages, ip, w.indices[:3])) == _lib.DH_EINVAL


def test_sequence_length_limit():
    """DH_MAX_SEQ_LEN tokens (8192 pages) plan; one page more is DH_EINVAL."""
    cfg = AttentionConfig(8, 2, 128)
    n = _lib.MAX_SEQ_LEN // 16
    ok = plan_inspect(cfg, n + 1, np.array([0, n], np.uint32), np.arange(n, dtype=np.uint32))
    assert ok["stats"]["total_pages"] == n
    with pytest.raises(DhError) as e:
        plan_inspect(cfg, n + 1, np.array([0, n + 1], np.uint32), np.arange(n + 1, dtype=np.uint32))
    assert e.value.status == _lib.DH_EINVAL


def test_direct_plan_selection():
    """Direct (merge-free) decode plans: flat plans of short sequences, or
    whose (sequence, KV head) workgroups alone fill the target; never with a
    shared segment, a group item, an empty sequence or DIRECT_OFF."""
    def direct(w, cascade=True, **kw):
        return plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices, cascade=cascade, **kw)["stats"]["direct"]
    short = workloads.custom([[1, 2], [3], [4, 5, 6, 7]], 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, 16)
    assert direct(short) == 1
    assert direct(short, direct=False) == 0
    assert direct(workloads.c1()) == 0                 # 32 pages: more, shorter chunks do better
    assert direct(workloads.c3(), cascade=False) == 1  # 64 x 8 workgroups fill the chip
    assert direct(workloads.c3()) == 0                 # shared prefixes
    assert direct(workloads.c4()) == 0                 # forked sequences share pages
    empty = workloads.custom([[1, 2], [], [3]], 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, 16)
    assert direct(empty) == 0
    # 32 query heads per KV head: runs of at most 16 pages stay wave items
    # (two row blocks), longer ones are group items
    many_heads = workloads.custom([[1, 2], [3]], 64, 2, 128, _lib.DTYPE_BF16, _lib.KV_BF16, 16)
    assert direct(many_heads) == 1
    long_many_heads = workloads.custom([list(range(1, 21)), [21]], 64, 2, 128, _lib.DTYPE_BF16, _lib.KV_BF16, 32)
    assert direct(long_many_heads) == 0


def test_flat_wave_chunk_by_list_schedule():
    """A plan of wave items only with work to spare takes the wave chunk whose
    heaviest-first schedule over the chip's wave slots ends first: C4 (256
    sequences of 32-256 FP8 pages) gets 96-page chunks (measured fastest of
    32 / 64 / 96 / 128 / 256), and every row still reads its pages once."""
    w = workloads.c4()
    plan = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices)
    st = plan["stats"]
    assert st["num_group_items"] == 0
    sizes = [int(it["npages"]) for it in plan["items"]]
    assert max(sizes) == 96 and st["num_items"] == 4120
    _check_cover(w, plan)
    # explicit options keep their meaning (no schedule estimate)
    fixed = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices, private_chunk_pages=32)
    assert max(int(it["npages"]) for it in fixed["items"]) <= 32


def test_short_shared_runs_stay_wave_items():
    """A shared run of at most 16 pages under at most 64 rows is read by wave
    items, one per 16-row block (C3's level-1 nodes: 8 pages, 16 leaves x 4
    heads); the 512-page root stays group items of 128 rows."""
    w = workloads.c3()
    plan = plan_inspect(_cfg(w), w.num_pool_pages, w.indptr, w.indices)
    st = plan["stats"]
    assert st["num_group_items"] == 256                  # root: 16 chunks x 8 heads x 2 row blocks
    groups = plan["items"][:st["num_group_items"]]
    assert all(int(it["nrows"]) == 128 and int(it["npages"]) == 32 for it in groups)
    waves = plan["items"][st["num_group_items"]:]
    assert max(int(it["nrows"]) for it in waves) == 16
    _check_cover(w, plan)
