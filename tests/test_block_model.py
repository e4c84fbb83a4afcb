"""Block model: the reference's integer tests, ported, plus a differential
property test of the C++ block model against the Python restatement.

Every test below named after a reference test follows it assertion for
assertion:
  BlockTable  crates/dendrite-core/src/cache/block_table.rs:112-316
  BlockPool   crates/dendrite-core/src/cache/pool.rs:120-272
  KvCache     crates/dendrite-core/src/cache/mod.rs:145-248 (+ proptests :251-365)
  TreeState   crates/dendrite-core/src/tree/state.rs:214-650
Each ported test runs twice: against the product, the C++ block model in
libdendrite_hip.so reached through dendrite_amd.cache (host code only: no GPU
is touched), and against the test oracle's pure-Python restatement
(oracle/block_model.py, through tests/_block_model_oracle_api.py), so the
reference's own assertions pin both.
"""
import pytest
from hypothesis import HealthCheck, given, settings, strategies as st

import dendrite_amd.cache as _product
from dendrite_amd import DhError
from dendrite_amd.cache import (BlockId, BlockPool, BlockTable, KvCache, KvCacheConfig, NodeId,
                                TreeState)
from oracle import block_model as ref

import _block_model_oracle_api as _oracle_api

_NAMES = ("BlockId", "BlockPool", "BlockTable", "KvCache", "KvCacheConfig", "NodeId", "TreeState")
_IMPLS = {
    "product": dict({n: getattr(_product, n) for n in _NAMES}, DhError=DhError),
    "oracle": dict({n: getattr(_oracle_api, n) for n in _NAMES}, DhError=_oracle_api.OracleError),
}
# The swap below is a plain rebinding of module names, so a fixture shared
# by every Hypothesis example is harmless.
_HC = [HealthCheck.function_scoped_fixture]


@pytest.fixture(autouse=True, params=sorted(_IMPLS))
def impl(request):
    """Binds the block-model names of this module to one implementation."""
    g = globals()
    saved = {n: g[n] for n in _IMPLS["product"]}
    g.update(_IMPLS[request.param])
    yield request.param
    g.update(saved)


# ---------------------------------------------------------------- BlockTable
def test_new_creates_empty_table():
    t = BlockTable.new(16)
    assert t.num_blocks() == 0 and t.num_tokens() == 0


def test_with_capacity_creates_empty_table_with_capacity():
    t = BlockTable.with_capacity(16, 10)
    assert t.num_blocks() == 0 and t.num_tokens() == 0


def test_push_adds_blocks():
    t = BlockTable(16)
    for b in (0, 5, 10):
        t.push(BlockId(b))
    assert t.num_blocks() == 3
    assert [t.get(i) for i in range(3)] == [0, 5, 10]


def test_get_returns_none_for_invalid_index():
    t = BlockTable(16)
    assert t.get(0) is None and t.get(100) is None


def test_block_for_token_calculates_correct_index():
    t = BlockTable(16)
    for b in (0, 1, 2):
        t.push(b)
    assert t.block_for_token(0) == 0 and t.block_for_token(15) == 0
    assert t.block_for_token(16) == 1 and t.block_for_token(31) == 1
    assert t.block_for_token(32) == 2
    assert t.block_for_token(48) is None


def test_set_updates_existing_block():
    t = BlockTable(16)
    t.push(0)
    t.push(1)
    t.set(0, 99)
    assert t.get(0) == 99 and t.get(1) == 1


def test_set_extends_table_if_needed():
    t = BlockTable(16)
    t.set(5, 42)
    assert t.num_blocks() == 6
    assert t.get(0) == BlockId.INVALID and t.get(4) == BlockId.INVALID
    assert t.get(5) == 42


def test_add_tokens_increments_count():
    t = BlockTable(16)
    t.add_tokens(10)
    assert t.num_tokens() == 10
    t.add_tokens(5)
    assert t.num_tokens() == 15


def test_set_num_tokens_updates_count():
    t = BlockTable(16)
    t.set_num_tokens(100)
    assert t.num_tokens() == 100
    t.set_num_tokens(50)
    assert t.num_tokens() == 50


def test_needs_new_block_empty_table():
    assert BlockTable(16).needs_new_block()


def test_needs_new_block_partial_block():
    t = BlockTable(16)
    t.push(0)
    t.set_num_tokens(10)
    assert not t.needs_new_block()


def test_needs_new_block_exactly_full():
    t = BlockTable(16)
    t.push(0)
    t.set_num_tokens(16)
    assert t.needs_new_block()


def test_needs_new_block_multiple_blocks():
    t = BlockTable(16)
    t.push(0)
    t.push(1)
    t.set_num_tokens(20)
    assert not t.needs_new_block()
    t.set_num_tokens(32)
    assert t.needs_new_block()


def test_fork_creates_shallow_copy():
    t = BlockTable(16)
    t.push(0)
    t.push(1)
    t.set_num_tokens(20)
    f = t.fork()
    assert f.num_blocks() == 2 and f.num_tokens() == 20
    assert f.get(0) == 0 and f.get(1) == 1
    assert f.blocks() == t.blocks()


def test_fork_is_independent():
    t = BlockTable(16)
    t.push(0)
    t.set_num_tokens(10)
    f = t.fork()
    f.push(99)
    f.set_num_tokens(20)
    assert t.num_blocks() == 1 and t.num_tokens() == 10


def test_clear_empties_table():
    t = BlockTable(16)
    t.push(0)
    t.push(1)
    t.set_num_tokens(32)
    t.clear()
    assert t.num_blocks() == 0 and t.num_tokens() == 0


def test_blocks_returns_all_block_ids():
    t = BlockTable(16)
    for b in (5, 10, 15):
        t.push(b)
    assert t.blocks() == [5, 10, 15]


# ----------------------------------------------------------------- BlockPool
def test_new_pool_has_all_blocks_free():
    assert BlockPool(10, 16).free_count() == 10


def test_allocate_returns_valid_block():
    p = BlockPool(10, 16)
    b = p.allocate()
    assert 0 <= b < 10
    assert p.free_count() == 9


def test_allocate_exhausts_pool():
    p = BlockPool(3, 16)
    for _ in range(3):
        p.allocate()
    assert p.free_count() == 0
    with pytest.raises(DhError):
        p.allocate()


def test_free_returns_block_to_pool():
    p = BlockPool(5, 16)
    b = p.allocate()
    assert p.free_count() == 4
    p.free(b)
    assert p.free_count() == 5


def test_free_invalid_block_returns_error():
    with pytest.raises(DhError):
        BlockPool(5, 16).free(BlockId(100))


def test_share_increments_refcount():
    p = BlockPool(5, 16)
    b = p.allocate()
    assert p.get_refcount(b) == 1
    p.share(b)
    assert p.get_refcount(b) == 2
    p.share(b)
    assert p.get_refcount(b) == 3


def test_share_invalid_block_returns_error():
    with pytest.raises(DhError):
        BlockPool(5, 16).share(BlockId(100))


def test_free_shared_block_decrements_refcount():
    p = BlockPool(5, 16)
    b = p.allocate()
    p.share(b)
    p.share(b)
    assert p.get_refcount(b) == 3 and p.free_count() == 4
    p.free(b)
    assert p.get_refcount(b) == 2 and p.free_count() == 4
    p.free(b)
    assert p.get_refcount(b) == 1 and p.free_count() == 4
    p.free(b)
    assert p.free_count() == 5


def test_copy_on_write_returns_same_if_not_shared():
    p = BlockPool(5, 16)
    b = p.allocate()
    assert p.copy_on_write(b) == b
    assert p.free_count() == 4


def test_copy_on_write_allocates_new_if_shared():
    p = BlockPool(5, 16)
    b = p.allocate()
    p.share(b)
    assert p.get_refcount(b) == 2
    nb = p.copy_on_write(b)
    assert nb != b
    assert p.get_refcount(b) == 1 and p.get_refcount(nb) == 1
    assert p.free_count() == 3


def test_copy_on_write_invalid_block_returns_error():
    with pytest.raises(DhError):
        BlockPool(5, 16).copy_on_write(BlockId(100))


def test_copy_on_write_fails_when_pool_exhausted():
    p = BlockPool(2, 16)
    b1 = p.allocate()
    p.allocate()
    p.share(b1)
    with pytest.raises(DhError):
        p.copy_on_write(b1)


def test_free_list_is_fifo():
    """pool.rs:40-45 pops the front, :58-59 pushes freed ids at the back."""
    p = BlockPool(4, 16)
    assert [p.allocate() for _ in range(3)] == [0, 1, 2]
    p.free(1)
    assert p.allocate() == 3
    assert p.allocate() == 1


def test_free_of_unallocated_block_is_an_error():
    """Deliberate deviation: the reference would drive the refcount of a free
    block to zero and queue its id twice; the port reports InvalidBlock."""
    p = BlockPool(4, 16)
    with pytest.raises(DhError):
        p.free(2)
    assert p.free_count() == 4


# ------------------------------------------------------------------- KvCache
def _cache(max_blocks, tokens_per_block=16):
    return KvCache(KvCacheConfig(num_layers=1, num_kv_heads=1, head_dim=64, max_blocks=max_blocks,
                                 tokens_per_block=tokens_per_block))


def test_new_cache_has_all_blocks_free():
    c = _cache(100)
    assert (c.free_blocks(), c.used_blocks(), c.total_blocks()) == (100, 0, 100)


def test_allocate_reduces_free_count():
    c = _cache(10)
    c.allocate_block()
    assert (c.free_blocks(), c.used_blocks()) == (9, 1)
    c.allocate_block()
    assert (c.free_blocks(), c.used_blocks()) == (8, 2)


def test_cache_free_returns_block_to_pool():
    c = _cache(10)
    b = c.allocate_block()
    assert c.free_blocks() == 9
    c.free_block(b)
    assert c.free_blocks() == 10


def test_share_and_free_refcount_behavior():
    c = _cache(10)
    b = c.allocate_block()
    c.share_block(b)
    c.share_block(b)
    c.free_block(b)
    assert c.free_blocks() == 9
    c.free_block(b)
    assert c.free_blocks() == 9
    c.free_block(b)
    assert c.free_blocks() == 10


def test_copy_on_write_unshared_returns_same():
    c = _cache(10)
    b = c.allocate_block()
    assert c.copy_on_write(b) == b and c.free_blocks() == 9


def test_copy_on_write_shared_allocates_new():
    c = _cache(10)
    b = c.allocate_block()
    c.share_block(b)
    assert c.copy_on_write(b) != b
    assert c.free_blocks() == 8


def test_config_accessible():
    cfg = _cache(50).config()
    assert cfg.max_blocks == 50 and cfg.tokens_per_block == 16


_cfg = st.tuples(st.integers(10, 99), st.sampled_from([8, 16, 32]))


@settings(max_examples=60, deadline=None, suppress_health_check=_HC)
@given(_cfg, st.integers(0, 49))
def test_invariant_block_count_consistency(cfg, alloc_count):
    c = _cache(*cfg)
    for _ in range(min(alloc_count, cfg[0])):
        c.allocate_block()
    assert c.free_blocks() + c.used_blocks() == c.total_blocks()


@settings(max_examples=60, deadline=None, suppress_health_check=_HC)
@given(_cfg, st.integers(1, 19))
def test_invariant_allocate_free_cycle(cfg, cycles):
    c = _cache(*cfg)
    initial = c.free_blocks()
    for _ in range(cycles):
        c.free_block(c.allocate_block())
    assert c.free_blocks() == initial


@settings(max_examples=60, deadline=None, suppress_health_check=_HC)
@given(_cfg, st.integers(0, 9))
def test_invariant_refcount_matches_shares(cfg, shares):
    c = _cache(*cfg)
    initial = c.free_blocks()
    b = c.allocate_block()
    for _ in range(shares):
        c.share_block(b)
    for _ in range(shares):
        c.free_block(b)
        assert c.free_blocks() == initial - 1
    c.free_block(b)
    assert c.free_blocks() == initial


@settings(max_examples=30, deadline=None, suppress_health_check=_HC)
@given(_cfg)
def test_invariant_cow_unshared_identity(cfg):
    c = _cache(*cfg)
    b = c.allocate_block()
    assert c.copy_on_write(b) == b


@settings(max_examples=30, deadline=None, suppress_health_check=_HC)
@given(_cfg)
def test_invariant_cow_shared_creates_new(cfg):
    c = _cache(*cfg)
    b = c.allocate_block()
    c.share_block(b)
    assert c.copy_on_write(b) != b


# ----------------------------------------------------------------- TreeState
def _tree(max_blocks=100):
    cache = _cache(max_blocks)
    return TreeState(cache, 16), cache


def test_new_creates_root_node():
    s, _ = _tree()
    info = s.get_node(NodeId.ROOT)
    assert info is not None
    assert info.id == NodeId.ROOT and info.parent is None and info.is_active
    assert info.num_children == 0


def test_fork_creates_child_node():
    s, _ = _tree()
    h = s.fork(NodeId.ROOT)
    assert h.node_id != NodeId.ROOT and h.depth == 1
    info = s.get_node(h.node_id)
    assert info.parent == NodeId.ROOT and info.is_active


def test_fork_increments_parent_child_count():
    s, _ = _tree()
    assert s.get_node(NodeId.ROOT).num_children == 0
    s.fork(NodeId.ROOT)
    assert s.get_node(NodeId.ROOT).num_children == 1
    s.fork(NodeId.ROOT)
    assert s.get_node(NodeId.ROOT).num_children == 2


def test_fork_from_invalid_node_returns_error():
    s, _ = _tree()
    with pytest.raises(DhError):
        s.fork(NodeId(99999))


def test_deep_fork_chain_calculates_depth():
    s, _ = _tree()
    nid = NodeId.ROOT
    for depth in range(1, 5):
        h = s.fork(nid)
        assert h.depth == depth
        nid = h.node_id


def test_multiple_forks_from_same_parent():
    s, _ = _tree()
    hs = [s.fork(NodeId.ROOT) for _ in range(3)]
    assert all(h.depth == 1 for h in hs)
    assert all(s.get_node(h.node_id).parent == NodeId.ROOT for h in hs)
    assert s.get_node(NodeId.ROOT).num_children == 3


def test_get_node_returns_none_for_invalid():
    s, _ = _tree()
    assert s.get_node(NodeId(99999)) is None


def test_release_deactivates_node():
    s, _ = _tree()
    h = s.fork(NodeId.ROOT)
    assert s.get_node(h.node_id).is_active
    s.release(h.node_id)
    after = s.get_node(h.node_id)
    assert after is None or not after.is_active


def test_release_decrements_parent_child_count():
    s, _ = _tree()
    h1, h2 = s.fork(NodeId.ROOT), s.fork(NodeId.ROOT)
    assert s.get_node(NodeId.ROOT).num_children == 2
    s.release(h1.node_id)
    assert s.get_node(NodeId.ROOT).num_children == 1
    s.release(h2.node_id)
    assert s.get_node(NodeId.ROOT).num_children == 0


def test_get_block_table_returns_blocks():
    s, _ = _tree()
    assert s.get_block_table(NodeId.ROOT) == []


def test_fork_handle_contains_correct_info():
    s, _ = _tree()
    h = s.fork(NodeId.ROOT)
    assert h.node_id.is_valid() and h.depth == 1 and h.num_tokens == 0


def test_append_token_updates_node():
    s, _ = _tree()
    h = s.fork(NodeId.ROOT)
    s.append_token(h.node_id, 42)
    assert s.get_node(h.node_id).num_tokens == 1


def test_append_token_allocates_blocks():
    s, _ = _tree()
    h = s.fork(NodeId.ROOT)
    assert s.get_block_table(h.node_id) == []
    s.append_token(h.node_id, 1)
    assert len(s.get_block_table(h.node_id)) == 1


def test_append_token_fills_block_before_allocating_new():
    s, _ = _tree()
    h = s.fork(NodeId.ROOT)
    for i in range(16):
        s.append_token(h.node_id, i)
    assert len(s.get_block_table(h.node_id)) == 1
    s.append_token(h.node_id, 16)
    assert len(s.get_block_table(h.node_id)) == 2


def test_append_token_to_invalid_node_fails():
    s, _ = _tree()
    with pytest.raises(DhError):
        s.append_token(NodeId(99999), 42)


def test_fork_after_tokens_inherits_blocks():
    s, _ = _tree()
    p = s.fork(NodeId.ROOT)
    for i in range(10):
        s.append_token(p.node_id, i)
    c = s.fork(p.node_id)
    assert c.num_tokens == 10
    assert s.get_block_table(p.node_id) == s.get_block_table(c.node_id)


def test_cow_triggered_when_forked_child_appends():
    s, cache = _tree()
    p = s.fork(NodeId.ROOT)
    for i in range(8):
        s.append_token(p.node_id, i)
    c = s.fork(p.node_id)
    before = cache.free_blocks()
    cow = s.append_token(c.node_id, 100)
    assert cache.free_blocks() <= before
    # The port also reports the copy the caller must make on the device.
    assert cow is not None
    old, new = cow
    assert old == s.get_block_table(p.node_id)[-1] and new == s.get_block_table(c.node_id)[-1]
    assert old != new


def test_multiple_forks_share_blocks():
    s, cache = _tree()
    p = s.fork(NodeId.ROOT)
    for i in range(32):
        s.append_token(p.node_id, i)
    used = cache.used_blocks()
    for _ in range(5):
        s.fork(p.node_id)
    assert cache.used_blocks() == used


def test_release_frees_blocks_when_no_references():
    s, cache = _tree()
    h = s.fork(NodeId.ROOT)
    for i in range(16):
        s.append_token(h.node_id, i)
    used = cache.used_blocks()
    assert used > 0
    s.release(h.node_id)
    assert cache.used_blocks() < used


def test_gc_preserves_nodes_with_active_children():
    s, _ = _tree()
    p = s.fork(NodeId.ROOT)
    c = s.fork(p.node_id)
    s.release(p.node_id)
    assert s.get_node(c.node_id) is not None


def test_tree_builds_correct_sequence():
    s, _ = _tree()
    a = s.fork(NodeId.ROOT)
    for i in range(1, 11):
        s.append_token(a.node_id, i)
    b = s.fork(a.node_id)
    for i in range(11, 21):
        s.append_token(b.node_id, i)
    assert s.get_node(a.node_id).num_tokens == 10
    assert s.get_node(b.node_id).num_tokens == 20


def test_branching_tree_structure():
    s, _ = _tree()
    base = s.fork(NodeId.ROOT)
    for i in range(5):
        s.append_token(base.node_id, i)
    b1, b2, b3 = (s.fork(base.node_id) for _ in range(3))
    for i in range(100, 105):
        s.append_token(b1.node_id, i)
    for i in range(200, 203):
        s.append_token(b2.node_id, i)
    for i in range(300, 310):
        s.append_token(b3.node_id, i)
    assert [s.get_node(b.node_id).num_tokens for b in (b1, b2, b3)] == [10, 8, 15]
    assert s.get_node(base.node_id).num_children == 3


# ----------------------------------------------- differential property test
_ops = st.lists(st.tuples(st.sampled_from(["fork", "append", "append", "append", "release"]),
                          st.integers(0, 10 ** 6)), min_size=1, max_size=120)


@settings(max_examples=120, deadline=None, suppress_health_check=_HC)
@given(_ops, st.integers(4, 64))
def test_tree_matches_python_restatement(impl, ops, max_blocks):
    """Random fork/append/release sequences drive the C++ tree and the Python
    restatement side by side; block tables, CoW pairs, refcounts, free counts
    and error outcomes must agree exactly."""
    if impl != "product":
        return          # product against oracle: one run covers it
    cache = _cache(max_blocks)
    tree = TreeState(cache, 16)
    rpool = ref.BlockPool(max_blocks, 16)
    rtree = ref.TreeState(rpool, 16)
    nodes = [0]
    for op, r in ops:
        nid = nodes[r % len(nodes)]
        if op == "fork":
            try:
                want = rtree.fork(nid)
            except ref.InvalidNode:
                with pytest.raises(DhError):
                    tree.fork(nid)
                continue
            got = tree.fork(nid)
            assert (got.node_id, got.depth, got.num_tokens) == want
            nodes.append(want[0])
        elif op == "append":
            try:
                want = rtree.append_token(nid, r)
            except (ref.InvalidNode, ref.OutOfMemory):
                with pytest.raises(DhError):
                    tree.append_token(nid, r)
                # The reference leaves a block pushed before a failed CoW in
                # place; both models must agree on that state too.
                continue
            got = tree.append_token(nid, r)
            assert got == want
        else:
            if nid == 0:
                continue
            rtree.release(nid)
            tree.release(nid)
        assert cache.free_blocks() == rpool.free_count()
        for n in set(nodes):
            if n in rtree.nodes:
                assert tree.get_block_table(n) == rtree.nodes[n].table.blocks
                assert tree.get_node(n).num_tokens == rtree.nodes[n].table.num_tokens
            else:
                assert tree.get_node(n) is None
        for b in range(max_blocks):
            assert cache.pool.get_refcount(b) == rpool.refcount[b]


def test_fork_below_a_collected_parent():
    """Releasing a node and then its only child collects the parent while the
    grandchild lives; a fork there counts depth up to the missing parent, as
    calculate_depth does (tree/state.rs:157-171)."""
    s, _ = _tree()
    a = s.fork(NodeId.ROOT).node_id
    b = s.fork(a).node_id
    c = s.fork(b).node_id
    s.release(a)
    s.release(b)                      # a: inactive, no children left -> collected
    assert s.get_node(a) is None and s.get_node(b) is not None
    h = s.fork(b)
    assert h.depth == 2
    assert s.get_node(c).parent == b
