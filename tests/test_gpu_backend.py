"""HipBackend, the AttentionBackend mirror (attention/backend.rs:61-97), and the
pool / merge entry points, through the C ABI on the GPU.

The ReferenceBackend tests of backend.rs:304-497 check shapes only (unseeded
randn); the ports below keep those assertions and add numerics against the
CPU oracle on the same seeded inputs.
"""
import numpy as np
import pytest
import torch

import oracle
from dendrite_amd import DhError, _lib
from dendrite_amd.backend import AttentionConfig, Backend, HipBackend, Pool
from dendrite_amd.cache import BlockId, BlockTable, KvCache, KvCacheConfig, NodeId, TreeState

pytestmark = pytest.mark.gpu


def _randn(shape, seed):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def _oracle_for(be: HipBackend, tables, queries, cfg: AttentionConfig):
    """Oracle output of the tables as the backend stores them."""
    ids = sorted({int(b) for t in tables for b in t.blocks() if b.is_valid() and int(b) in be.page_len})
    data = np.stack([be.pool.read_page(p)[0] for p in ids]) if ids else np.zeros((0, be.pool.page_bytes),
                                                                                 np.uint8)
    pv = oracle.PoolView(np.array(ids, dtype=np.uint32), data, None, be.pool.num_pages, be.pool.kv_format,
                         be.pool.num_kv_heads, be.pool.head_dim)
    indptr, indices, lpl = be._csr(tables)
    q = np.stack([x.reshape(cfg.num_heads, cfg.head_dim).float().numpy() for x in queries])
    return oracle.decode(pv, q, _lib.DTYPE_F32, cfg.num_heads, cfg.scale, cfg.gqa_mapping, indptr, indices,
                         lpl)


def _store_block(be, block, seed, n=16, hkv=4, d=64):
    be.append_kv(_randn((1, hkv, n, d), seed), _randn((1, hkv, n, d), seed + 1),
                 BlockTable.from_blocks([block]), 0)


def test_reference_backend_decode_empty_cache():
    be = HipBackend(num_pages=16, num_kv_heads=4, head_dim=64, kv_format=_lib.KV_F32)
    cfg = AttentionConfig(4, 4, 64)
    q = _randn((1, 4, 1, 64), 1)
    out = be.decode(q, BlockTable(16), cfg)
    assert tuple(out.shape) == tuple(q.shape)
    assert not out.abs().sum().item()


def test_reference_backend_decode_with_cache():
    be = HipBackend(num_pages=16, num_kv_heads=4, head_dim=64, kv_format=_lib.KV_F32)
    cfg = AttentionConfig(4, 4, 64)
    _store_block(be, 0, 10)
    t = BlockTable(16)
    t.push(BlockId(0))
    q = _randn((1, 4, 1, 64), 2)
    out = be.decode(q, t, cfg)
    assert tuple(out.shape) == tuple(q.shape)
    want = _oracle_for(be, [t], [q], cfg)
    assert np.max(np.abs(out.cpu().reshape(1, 4, 64).numpy() - want)) < 1e-4


def test_reference_backend_decode_batch():
    be = HipBackend(num_pages=16, num_kv_heads=4, head_dim=64, kv_format=_lib.KV_F32)
    cfg = AttentionConfig(4, 4, 64)
    _store_block(be, 0, 20)
    _store_block(be, 1, 30)
    t1, t2 = BlockTable.from_blocks([0]), BlockTable.from_blocks([1])
    qs = [_randn((1, 4, 1, 64), 3), _randn((1, 4, 1, 64), 4)]
    outs = be.decode_batch(qs, [t1, t2], cfg)
    assert len(outs) == 2
    assert all(tuple(o.shape) == tuple(q.shape) for o, q in zip(outs, qs))
    want = _oracle_for(be, [t1, t2], qs, cfg)
    got = np.stack([o.cpu().reshape(4, 64).numpy() for o in outs])
    assert np.max(np.abs(got - want)) < 1e-4


def test_reference_backend_append_kv_single_token():
    be = HipBackend(num_pages=16, num_kv_heads=4, head_dim=64, kv_format=_lib.KV_F32)
    cfg = AttentionConfig(4, 4, 64)
    k, v = _randn((1, 4, 1, 64), 5), _randn((1, 4, 1, 64), 6)
    t = BlockTable.from_blocks([0], num_tokens=1)
    be.append_kv(k, v, t, 0)
    assert be.page_len[0] == 1
    out = be.decode(_randn((1, 4, 1, 64), 7), t, cfg)
    # one token: the output is its V row, exactly
    assert np.array_equal(out.cpu().reshape(4, 64).numpy(), v.reshape(4, 64).numpy())


@pytest.mark.parametrize("kvf", [_lib.KV_BF16, _lib.KV_F16, _lib.KV_F32])
def test_backend_tree_decode_matches_oracle(kvf):
    """A TreeState-built tree (fork + append with CoW) decoded through the
    backend: GQA 8/2, partial last pages, shared prefixes."""
    import torch
    hq, hkv, d = 8, 2, 128
    be = HipBackend(num_pages=128, num_kv_heads=hkv, head_dim=d, kv_format=kvf)
    cache = KvCache(KvCacheConfig(num_layers=1, num_kv_heads=hkv, head_dim=d, max_blocks=128))
    tree = TreeState(cache, 16)
    seed = [100]

    def append(node, n):
        for _ in range(n):
            cow = tree.append_token(node, 0)
            if cow is not None:                      # CoW: copy the shared page's data first
                be.pool.copy_page(int(cow[0]), int(cow[1]))
                be.page_len[int(cow[1])] = be.page_len.get(int(cow[0]), 0)
            blocks = tree.get_block_table(node)
            pos = tree.get_node(node).num_tokens - 1
            seed[0] += 2
            be.append_kv(_randn((1, hkv, 1, d), seed[0]), _randn((1, hkv, 1, d), seed[0] + 1),
                         BlockTable.from_blocks(blocks), pos)

    base = tree.fork(NodeId.ROOT).node_id
    append(base, 40)                                 # 2.5 pages
    leaves = []
    for i in range(3):
        c = tree.fork(base).node_id
        append(c, 5 + 11 * i)
        leaves.append(c)
    tables = [BlockTable.from_blocks(tree.get_block_table(n), tree.get_node(n).num_tokens) for n in leaves]
    cfg = AttentionConfig(hq, hkv, d)
    tdt = {_lib.KV_BF16: torch.bfloat16, _lib.KV_F16: torch.float16, _lib.KV_F32: torch.float32}[kvf]
    qs = [_randn((1, hq, 1, d), 900 + i).to(tdt) for i in range(3)]
    outs = be.decode_batch(qs, tables, cfg)
    want = _oracle_for(be, tables, [q.to(torch.float32) for q in qs], cfg)
    got = np.stack([o.float().cpu().reshape(hq, d).numpy() for o in outs])
    tol = 1e-4 if kvf == _lib.KV_F32 else 2e-2
    assert np.max(np.abs(got - want)) < tol


def test_prefill_errors():
    """prefill takes f32 / bf16 / f16 queries (else DH_EUNSUPPORTED) and key /
    value of the query's batch and length (else DH_EINVAL)."""
    import torch
    be = HipBackend(num_pages=4, num_kv_heads=4, head_dim=64)
    cfg = AttentionConfig(4, 4, 64)
    q = torch.zeros(1, 4, 8, 64, dtype=torch.float64)
    with pytest.raises(DhError) as e:
        be.prefill(q, q, q, BlockTable(16), cfg)
    assert e.value.status == _lib.DH_EUNSUPPORTED
    qb = q.to(torch.bfloat16)
    with pytest.raises(DhError) as e:
        be.prefill(qb, qb[:, :, :5], qb[:, :, :5], BlockTable(16), cfg)
    assert e.value.status == _lib.DH_EINVAL


@pytest.mark.parametrize("kvf", [_lib.KV_BF16, _lib.KV_FP8_E4M3, _lib.KV_MXFP8])
def test_pool_write_copy_read_roundtrip(backend, kvf):
    """write_pages / read_page / copy_page (the CoW data copy the reference
    leaves as a TODO, cache/pool.rs:90) and write_tokens at an offset."""
    from dendrite_amd import workloads
    w = workloads.random_tree(5, 8, 2, 64, _lib.DTYPE_BF16, kvf, n_leaves=3, pool_pages=64)
    pool = Pool(backend, 64, 2, 64, kvf)
    ids = w.page_ids()[:4]
    data, scales = w.make_pages(ids)
    pool.write_pages(ids, data, scales)
    for i, p in enumerate(ids):
        d, s = pool.read_page(int(p))
        assert np.array_equal(d, data[i].reshape(-1).view(np.uint8))
        if scales is not None:
            assert np.array_equal(s, scales[i].reshape(-1).view(np.uint8))
    free = next(p for p in range(64) if p not in set(int(x) for x in ids))
    pool.copy_page(int(ids[2]), free)
    backend.synchronize()
    d2, s2 = pool.read_page(free)
    assert np.array_equal(d2, data[2].reshape(-1).view(np.uint8))
    if scales is not None:
        assert np.array_equal(s2, scales[2].reshape(-1).view(np.uint8))
    if kvf == _lib.KV_BF16:
        rng = np.random.Generator(np.random.PCG64(1))
        k = rng.integers(0, 2 ** 16, size=(2, 5, 64), dtype=np.uint16)
        v = rng.integers(0, 2 ** 16, size=(2, 5, 64), dtype=np.uint16)
        pool.write_tokens(free, 7, k, v)
        d3, _ = pool.read_page(free)
        page = d3.view(np.uint16).reshape(2, 2, 16, 64)
        ref = data[2].reshape(-1).view(np.uint16).reshape(2, 2, 16, 64).copy()
        ref[0, :, 7:12] = k
        ref[1, :, 7:12] = v
        assert np.array_equal(page, ref)


def test_merge_states_matches_closed_form(backend):
    import torch
    n, d = 37, 64
    g = torch.Generator().manual_seed(3)
    oa, ob = torch.randn(n, d, generator=g), torch.randn(n, d, generator=g)
    la, lb = torch.randn(n, generator=g) * 4, torch.randn(n, generator=g) * 4
    la[0] = lb[0] = float("-inf")                # two empty sides
    la[1] = float("-inf")                        # one empty side
    lb[2] = float("-inf")
    dev = [x.cuda() for x in (oa, la, ob, lb)]
    oo, lo = torch.empty(n, d, device="cuda"), torch.empty(n, device="cuda")
    _lib.check(_lib.lib().dh_merge_states(*(x.data_ptr() for x in dev), oo.data_ptr(), lo.data_ptr(),
                                          n, d, None))
    torch.cuda.synchronize()
    oo, lo = oo.cpu().numpy(), lo.cpu().numpy()
    assert not np.any(oo[0]) and lo[0] == float("-inf")
    assert np.allclose(oo[1], ob[1].numpy(), atol=1e-6) and np.isclose(lo[1], lb[1].item())
    assert np.allclose(oo[2], oa[2].numpy(), atol=1e-6) and np.isclose(lo[2], la[2].item())
    for i in range(3, n):
        for k in range(0, d, 7):
            o, l = oracle.merge(oa[i, k].item(), la[i].item(), ob[i, k].item(), lb[i].item())
            assert abs(oo[i, k] - o) < 1e-5 and abs(lo[i] - l) < 1e-5


def test_decode_rejects_bad_workspace(backend):
    import torch
    from dendrite_amd import workloads
    from dendrite_amd.backend import DecodePlan, decode_batch
    w = workloads.c2(branches=2, prefix_pages=4, suffix_pages=2, pool_pages=64)
    pool = Pool(backend, w.num_pool_pages, w.hkv, w.d, w.kv_format)
    plan = DecodePlan(backend, w.attention_config(), pool, w.indptr, w.indices)
    q = torch.zeros(w.batch, w.hq, w.d, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(DhError) as e:
        decode_batch(plan, q, out, small)
    assert e.value.status == _lib.DH_EINVAL


@pytest.mark.parametrize("bad", [0.0, -1.0, float("nan"), float("inf")])
def test_fp8_block_scales_must_be_positive(backend, bad):
    """FP8 E4M3 block scales are finite and > 0 (the quantiser's amax / 448,
    1 for an all-zero block); others are rejected on write, before any copy."""
    hkv, d = 2, 128
    pool = Pool(backend, 8, hkv, d, _lib.KV_FP8_E4M3)
    data = np.zeros((1, pool.page_bytes), dtype=np.uint8)
    scales = np.ones((1, 2 * hkv), dtype=np.float32)
    pool.write_pages([3], data, scales.view(np.uint8))
    scales[0, 1] = bad
    with pytest.raises(DhError) as e:
        pool.write_pages([3], data, scales.view(np.uint8))
    assert e.value.status == _lib.DH_EINVAL
    k = np.zeros((hkv, 16, d), dtype=np.uint8)
    with pytest.raises(DhError):
        pool.write_tokens(3, 0, k, k, k_scale=np.array([1.0, bad], np.float32),
                          v_scale=np.ones(hkv, np.float32))
    _, s = pool.read_page(3)
    assert np.array_equal(s.view(np.float32), np.ones(2 * hkv, np.float32))


def test_store_get_and_clear():
    """store_kv / get_kv round trip (bf16 and f32 pools), overwrite
    semantics, and clear_cache: afterwards decode sees no KV (zeros, as
    ReferenceBackend with an empty cache, backend.rs:218-222)."""
    for fmt, dt in ((_lib.KV_BF16, torch.bfloat16), (_lib.KV_F32, torch.float32)):
        be = HipBackend(num_pages=8, num_kv_heads=2, head_dim=64, kv_format=fmt)
        g = torch.Generator().manual_seed(5)
        k = torch.randn(1, 2, 11, 64, generator=g).to(dt)
        v = torch.randn(1, 2, 11, 64, generator=g).to(dt)
        assert be.get_kv(3) is None
        be.store_kv(3, k, v)
        gk, gv = be.get_kv(3)
        assert torch.equal(gk, k) and torch.equal(gv, v)
        be.store_kv(3, k[:, :, :5], v[:, :, :5])            # overwrite: 5 tokens now
        gk, gv = be.get_kv(3)
        assert gk.shape[2] == 5 and torch.equal(gk, k[:, :, :5]) and torch.equal(gv, v[:, :, :5])
        cfg = AttentionConfig(8, 2, 64)
        cfg.q_dtype = _lib.DTYPE_BF16 if fmt == _lib.KV_BF16 else _lib.DTYPE_F32
        q = torch.randn(1, 8, 1, 64, generator=g).to(dt)
        assert be.decode(q, BlockTable.from_blocks([3]), cfg).abs().sum() > 0
        be.clear_cache()
        assert be.get_kv(3) is None
        assert torch.count_nonzero(be.decode(q, BlockTable.from_blocks([3]), cfg)) == 0


# ------------------------- the reference's own backend tests (backend.rs:346-415)
def test_reference_backend_new():
    backend = HipBackend.new(num_pages=4, num_kv_heads=4, head_dim=64)
    assert backend.page_len == {}


def test_reference_backend_store_kv():
    import torch
    backend = HipBackend.new(num_pages=4, num_kv_heads=4, head_dim=64, kv_format=_lib.KV_F32)
    key = torch.randn(1, 4, 16, 64)
    value = torch.randn(1, 4, 16, 64)
    backend.store_kv(0, key, value)
    assert backend.get_kv(0) is not None


def test_reference_backend_clear_cache():
    import torch
    backend = HipBackend.new(num_pages=4, num_kv_heads=4, head_dim=64, kv_format=_lib.KV_F32)
    backend.store_kv(0, torch.randn(1, 4, 16, 64), torch.randn(1, 4, 16, 64))
    assert backend.page_len
    backend.clear_cache()
    assert not backend.page_len


def test_reference_backend_prefill():
    import torch
    backend = HipBackend.new(num_pages=4, num_kv_heads=4, head_dim=64)
    config = AttentionConfig(4, 4, 64)
    query, key, value = (torch.randn(1, 4, 8, 64) for _ in range(3))
    output = backend.prefill(query, key, value, BlockTable(16), config)
    assert tuple(output.shape) == tuple(query.shape)


def test_reference_backend_prefill_gqa():
    import torch
    backend = HipBackend.new(num_pages=4, num_kv_heads=2, head_dim=64)
    config = AttentionConfig(8, 2, 64)
    query = torch.randn(1, 8, 4, 64)
    key, value = torch.randn(1, 2, 4, 64), torch.randn(1, 2, 4, 64)
    output = backend.prefill(query, key, value, BlockTable(16), config)
    assert tuple(output.shape) == tuple(query.shape)


@pytest.mark.parametrize("kvf", [_lib.KV_F32, _lib.KV_FP8_E4M3])
def test_append_kv_leaves_no_unwritten_tokens(kvf):
    """append_kv writes at offset position % 16, so it must never leave
    tokens in front of the write unwritten: after clear_cache (which forgets
    every block but keeps the pool's bytes), an append at position 17 into a
    block holding nothing is refused; appends from the block's front are
    accepted, and decode then sees exactly the tokens written."""
    hkv, d = 2, 64
    be = HipBackend(num_pages=8, num_kv_heads=hkv, head_dim=d, kv_format=kvf)
    table = BlockTable.from_blocks([3, 5], num_tokens=18)
    be.append_kv(_randn((1, hkv, 16, d), 40), _randn((1, hkv, 16, d), 41), table, 0)
    be.append_kv(_randn((1, hkv, 2, d), 42), _randn((1, hkv, 2, d), 43), table, 16)
    be.clear_cache()
    with pytest.raises(DhError) as e:
        be.append_kv(_randn((1, hkv, 1, d), 44), _randn((1, hkv, 1, d), 45), table, 17)
    assert e.value.status == _lib.DH_EUNSUPPORTED
    assert 5 not in be.page_len
    # refill from the front: token 16 then 17 of block 5 (block 3 stays forgotten)
    v16, v17 = _randn((1, hkv, 1, d), 47), _randn((1, hkv, 1, d), 49)
    be.append_kv(_randn((1, hkv, 1, d), 46), v16, table, 16)
    be.append_kv(_randn((1, hkv, 1, d), 48), v17, table, 17)
    assert be.page_len[5] == 2 and 3 not in be.page_len
    if kvf == _lib.KV_F32:
        cfg = AttentionConfig(hkv, hkv, d)
        cfg.q_dtype = _lib.DTYPE_F32
        cfg.kv_format = kvf
        q = torch.zeros((1, hkv, 1, d))          # zero query: equal weights over the tokens seen
        out = be.decode(q, table, cfg).cpu().reshape(hkv, d).numpy()
        want = 0.5 * (v16 + v17).reshape(hkv, d).numpy()
        assert np.max(np.abs(out - want)) < 1e-6


def test_trait_decode_reuses_and_patches_its_plan():
    """decode_batch through the trait with tables that grow one token per
    step (append_kv + add_tokens; a new block every 16 tokens) and a
    copy-on-write of a last block: the cached plan is reused between page
    boundaries, patched in place at them (dh_plan_update) and rebuilt only
    when a list changes elsewhere; every step matches the oracle."""
    import torch
    hq, hkv, d = 16, 4, 64
    be = HipBackend(num_pages=256, num_kv_heads=hkv, head_dim=d)
    cfg = AttentionConfig(hq, hkv, d)
    prefix = [1, 2, 3]
    for i, b in enumerate(prefix):
        _store_block(be, b, 100 + 2 * i, hkv=hkv, d=d)
    tables, pos, nxt = [], [], [10]
    for leaf in range(4):
        n0 = 5 + 3 * leaf
        t = BlockTable.from_blocks(prefix + [nxt[0]], num_tokens=48 + n0)
        be.append_kv(_randn((1, hkv, n0, d), 200 + 2 * leaf), _randn((1, hkv, n0, d), 201 + 2 * leaf), t, 48)
        tables.append(t)
        pos.append(48 + n0)
        nxt[0] += 1
    base = _randn((4, hq, d), 7).to(torch.bfloat16).cuda()
    queries = [base[i].view(1, hq, 1, d) for i in range(4)]

    def check(step):
        outs = be.decode_batch(queries, tables, cfg)
        got = np.stack([o.float().cpu().reshape(hq, d).numpy() for o in outs])
        want = _oracle_for(be, tables, [q.cpu() for q in queries], cfg)
        err = float(np.max(np.abs(got - want)))
        print(f"[case] trait step {step}: max abs err {err:.3e}", flush=True)
        assert err < 2e-2, step

    seed = 300
    for step in range(40):
        check(step)
        for i, t in enumerate(tables):
            if pos[i] % 16 == 0:
                t.push(nxt[0])
                nxt[0] += 1
            seed += 2
            be.append_kv(_randn((1, hkv, 1, d), seed), _randn((1, hkv, 1, d), seed + 1), t, pos[i])
            t.add_tokens(1)
            pos[i] += 1
    built, patched, reused = be.plans_built, be.plans_patched, be.plans_reused
    print(f"[case] trait plans: built {built}, patched {patched}, reused {reused}", flush=True)
    # leaves start 5, 8, 11, 14 tokens into their page: each crosses two or
    # three page boundaries in 40 steps, at different steps
    assert built == 1 and patched >= 8 and built + patched + reused == 40
    # copy-on-write of leaf 0's partial last block: REPLACE_LAST
    last = int(tables[0].block_ids()[-1])
    be.pool.copy_page(last, nxt[0])
    be.page_len[nxt[0]] = be.page_len[last]
    tables[0].set(tables[0].num_blocks() - 1, nxt[0])
    check("cow")
    assert be.plans_built == 1 and be.plans_patched == patched + 1
    # a middle block replaced: a new plan
    tables[1].set(1, 4)
    _store_block(be, 4, 400, hkv=hkv, d=d)
    check("middle")
    assert be.plans_built == 2
