"""In-place plan updates (dh_plan_update) against the CPU oracle.

A decode plan takes the page-list changes of a decode step without being
rebuilt: a page appended to a sequence (TreeState::append_token on a block
boundary, tree/state.rs:87-113) and the replacement of a shared partial last
page by its copy-on-write copy.  Checked here:
- TreeDecoder over a TreeState: a prompt, forks (also at a partial block, so
  the next append copies on write), many steps of one token per leaf with
  random K/V; every step's decode against the oracle (oracle_decode, pinned in
  test_oracle.py) on the tree's block tables at that step; most steps patch
  the plan, forks rebuild it.  Run over the patched item kinds: wave-item
  tails (4 query heads per KV head), group-item tails (24 per KV head, so a
  sequence's rows exceed one 16-row wave item), FP8 E4M3 block-scale and
  MXFP8 pages, f32 queries (the f32 kernel), and head_dim 64 / 128 / 256;
- the reserved room: 16 appends to one sequence fit, the 17th does not and
  leaves the plan as it was;
- argument errors, and prefill plans refused.
Tolerance: 2e-2 beyond bf16 output rounding (1e-4 for f32), as for every decode.
"""
import numpy as np
import pytest
import torch

import oracle
from dendrite_amd import DhError, _lib
from dendrite_amd.backend import (AttentionConfig, Backend, DecodePlan, Pool, PrefillPlan, TreeDecoder,
                                  decode_batch)
from dendrite_amd.cache import KvCache, KvCacheConfig, NodeId, TreeState
from tests._helpers import TOL, excess_err

pytestmark = pytest.mark.gpu

HKV, D, HQ = 2, 64, 8


# E4M3 block scale of every token written to an FP8 page: one fixed value,
# so single-token writes (each passing the page's scale) keep a page's codes
# consistent.
FP8_SCALE = 1.0 / 64


class Mirror:
    """The pool's pages (raw bytes in the pool format) on the host, for the
    oracle; tokens are written one at a time, encoded here."""

    def __init__(self, pool: Pool, fmt=_lib.KV_BF16, hkv=HKV, d=D):
        self.pool, self.fmt, self.hkv, self.d = pool, fmt, hkv, d
        self.eb = {_lib.KV_BF16: 2, _lib.KV_F16: 2, _lib.KV_F32: 4}.get(fmt, 1)
        self.data = np.zeros((pool.num_pages, 2, hkv, 16, d * self.eb), np.uint8)
        if fmt == _lib.KV_FP8_E4M3:
            self.scales = np.zeros((pool.num_pages, 2, hkv), np.float32)
        elif fmt == _lib.KV_MXFP8:
            self.scales = np.zeros((pool.num_pages, 2, hkv, 16, d // 32), np.uint8)
        else:
            self.scales = None

    @staticmethod
    def _e4m3(x):
        return torch.from_numpy(np.clip(x, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    def write(self, page, off, rng):
        hkv, d = self.hkv, self.d
        x = rng.standard_normal((2, hkv, 1, d)).astype(np.float32)
        ks = vs = None
        if self.fmt == _lib.KV_F32:
            raw = x.view(np.uint8).reshape(2, hkv, 1, -1)
        elif self.fmt == _lib.KV_BF16:
            raw = torch.from_numpy(x).to(torch.bfloat16).view(torch.uint8).numpy().reshape(2, hkv, 1, -1)
        elif self.fmt == _lib.KV_FP8_E4M3:
            raw = self._e4m3(x / FP8_SCALE)
            ks = vs = np.full(hkv, FP8_SCALE, np.float32)
            self.scales[page] = FP8_SCALE
        else:   # MXFP8: per 32 elements along head_dim, 2^(floor(log2 amax) - 8)
            g = x.reshape(2, hkv, 1, d // 32, 32)
            amax = np.abs(g).max(axis=4)
            e = np.where(amax > 0, np.floor(np.log2(np.maximum(amax, 1e-30))) - 8, -127).clip(-127, 127)
            raw = self._e4m3((g / np.ldexp(1.0, e.astype(np.int64))[..., None]).astype(np.float32)).reshape(2, hkv, 1, d)
            sc = (e + 127).astype(np.uint8)                        # [2][hkv][1][d/32]
            ks, vs = sc[0], sc[1]
            self.scales[page, :, :, off:off + 1] = sc
        self.pool.write_tokens(page, off, raw[0], raw[1], ks, vs)
        self.data[page, :, :, off:off + 1] = raw

    def copy(self, src, dst):
        self.data[dst] = self.data[src]
        if self.scales is not None:
            self.scales[dst] = self.scales[src]

    def view(self):
        n = self.pool.num_pages
        sc = None if self.scales is None else self.scales.view(np.uint8).reshape(n, -1)
        return oracle.PoolView(np.arange(n, dtype=np.uint32), self.data.reshape(n, -1), sc, n, self.fmt,
                               self.hkv, self.d)


def _oracle(mirror, cfg, q, tables, lpl, hq=HQ):
    indptr = np.cumsum([0] + [len(t) for t in tables]).astype(np.uint32)
    indices = np.array([b for t in tables for b in t], dtype=np.uint32)
    return oracle.decode(mirror.view(), q.float().cpu().numpy(), _lib.DTYPE_F32, hq, cfg.scale, cfg.gqa_mapping,
                         indptr, indices, np.asarray(lpl, np.int32))


def _q(rng, n, hq=HQ, d=D, dtype=torch.bfloat16):
    return torch.from_numpy(rng.standard_normal((n, hq, d)).astype(np.float32)).to(dtype).to("cuda:0")


# (query heads, KV heads, head_dim, KV format, query dtype, decode steps)
_TREE_CASES = {
    "bf16-r4-d64": (HQ, HKV, D, _lib.KV_BF16, _lib.DTYPE_BF16, 70),
    "bf16-r24-d128": (48, 2, 128, _lib.KV_BF16, _lib.DTYPE_BF16, 40),
    "bf16-r4-d256": (8, 2, 256, _lib.KV_BF16, _lib.DTYPE_BF16, 40),
    "fp8-r4-d128": (8, 2, 128, _lib.KV_FP8_E4M3, _lib.DTYPE_BF16, 40),
    "mxfp8-r8-d128": (16, 2, 128, _lib.KV_MXFP8, _lib.DTYPE_BF16, 40),
    "f32-r4-d64": (8, 2, 64, _lib.KV_F32, _lib.DTYPE_F32, 40),
}


@pytest.mark.parametrize("case", sorted(_TREE_CASES))
def test_tree_decoder_patches_the_plan_step_after_step(backend, case):
    hq, hkv, d, fmt, qdt, nsteps = _TREE_CASES[case]
    rng = np.random.default_rng(11)
    num_pages = 192
    pool = Pool(backend, num_pages, hkv, d, fmt)
    mirror = Mirror(pool, fmt, hkv, d)
    tree = TreeState(KvCache(KvCacheConfig(num_kv_heads=hkv, head_dim=d, max_blocks=num_pages)), 16)
    cfg = AttentionConfig(hq, hkv, d)
    cfg.q_dtype = qdt
    cfg.kv_format = fmt
    tdt = torch.float32 if qdt == _lib.DTYPE_F32 else torch.bfloat16
    dec = TreeDecoder(backend, pool, tree, cfg, [NodeId.ROOT])

    def append(i):
        before = tree.get_block_table(dec.leaves[i]) or []
        page, off = dec.append_token(i, int(rng.integers(0, 32000)))
        after = tree.get_block_table(dec.leaves[i])
        if before and after[-1] != before[-1] and len(after) == len(before):   # copy on write
            mirror.copy(int(before[-1]), int(after[-1]))
        mirror.write(page, off, rng)

    def step():
        q = _q(rng, len(dec.leaves), hq, d, tdt)
        out = dec.decode(q)
        torch.cuda.synchronize()
        ref = _oracle(mirror, cfg, q, dec.tables(), dec.last_page_len(), hq)
        err = excess_err(out.float().cpu().numpy(), ref, qdt)
        assert err <= TOL[qdt], f"{case}: step with {len(dec.leaves)} leaves: {err}"

    for _ in range(37):                      # prompt: two full pages and five tokens
        append(0)
    step()
    for _ in range(3):                       # forks at a partial block
        dec.fork(0)
    step()
    for s in range(nsteps):
        for i in range(len(dec.leaves)):
            append(i)
            if (s + i) % 5 == 0:             # leaves drift apart in length
                append(i)
        if s in (9, min(40, nsteps - 10)):   # a fork in the middle of decoding
            dec.fork(1 + s % 3)
        step()
    assert dec.plans_built >= 4
    assert dec.plans_patched >= (10 if nsteps >= 70 else 5), (dec.plans_built, dec.plans_patched)


def _pages_plan(backend, pool, cfg, tables):
    indptr = np.cumsum([0] + [len(t) for t in tables]).astype(np.uint32)
    indices = np.array([b for t in tables for b in t], dtype=np.uint32)
    return DecodePlan(backend, cfg, pool, indptr, indices)


def _decode(plan, q, lpl):
    out = torch.empty_like(q)
    lp = torch.from_numpy(np.asarray(lpl, np.int32)).to("cuda:0")
    decode_batch(plan, q, out, plan.workspace(), lp)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_room_for_sixteen_appends_then_a_new_plan(backend):
    rng = np.random.default_rng(12)
    pool = Pool(backend, 64, HKV, D, _lib.KV_BF16)
    mirror = Mirror(pool)
    for p in range(64):
        for t in range(16):
            mirror.write(p, t, rng)
    cfg = AttentionConfig(HQ, HKV, D)
    tables = [[0, 1, 2, 3], [0, 1, 5], [7]]
    plan = _pages_plan(backend, pool, cfg, tables)
    lpl = [16, 9, 3]
    q = _q(rng, 3)
    before = plan.stats()
    for k in range(16):
        assert plan.update([(0, _lib.PLAN_APPEND, 20 + k)])
        tables[0].append(20 + k)
    assert plan.stats()["total_pages"] == before["total_pages"] + 16
    got = _decode(plan, q, lpl)
    ref = _oracle(mirror, cfg, q, tables, lpl)
    assert excess_err(got, ref, _lib.DTYPE_BF16) <= TOL[_lib.DTYPE_BF16]
    # no room left: nothing changes, not even the events that would fit
    assert not plan.update([(2, _lib.PLAN_APPEND, 40), (0, _lib.PLAN_APPEND, 41)])
    assert np.array_equal(_decode(plan, q, lpl), got)
    # the last page replaced (copy on write), in a batch with an append
    assert plan.update([(1, _lib.PLAN_REPLACE_LAST, 44), (2, _lib.PLAN_APPEND, 45), (2, _lib.PLAN_APPEND, 46)])
    tables[1][-1] = 44
    tables[2] += [45, 46]
    lpl = [16, 9, 12]
    got = _decode(plan, q, lpl)
    ref = _oracle(mirror, cfg, q, tables, lpl)
    assert excess_err(got, ref, _lib.DTYPE_BF16) <= TOL[_lib.DTYPE_BF16]
    # a new plan on the same lists agrees
    fresh = _decode(_pages_plan(backend, pool, cfg, tables), q, lpl)
    assert excess_err(fresh, ref, _lib.DTYPE_BF16) <= TOL[_lib.DTYPE_BF16]


def test_update_errors(backend):
    pool = Pool(backend, 16, HKV, D, _lib.KV_BF16)
    cfg = AttentionConfig(HQ, HKV, D)
    plan = _pages_plan(backend, pool, cfg, [[0, 1], [2], []])
    for ev in ([(3, _lib.PLAN_APPEND, 4)], [(0, _lib.PLAN_APPEND, 16)], [(0, 7, 4)],
               [(0, _lib.PLAN_APPEND, _lib.INVALID_PAGE)]):
        with pytest.raises(DhError) as e:
            plan.update(ev)
        assert e.value.status == _lib.DH_EINVAL
    assert plan.update([])                          # nothing to do
    assert not plan.update([(2, _lib.PLAN_APPEND, 4)])   # a sequence without pages
    pcfg = AttentionConfig(HQ, HKV, D)
    pcfg.q_dtype = _lib.DTYPE_BF16
    pre = PrefillPlan(backend, pcfg, pool, np.array([0, 2], np.uint32), np.array([0, 1], np.uint32),
                      np.array([20], np.uint32), np.array([4], np.uint32), causal=True)
    with pytest.raises(DhError) as e:
        pre.update([(0, _lib.PLAN_APPEND, 3)])
    assert e.value.status == _lib.DH_EUNSUPPORTED


def test_plan_from_tree_equals_plan_from_its_tables(backend):
    """dh_plan_create_tree reads the same page lists a caller would pass in
    CSR form (outputs bit-identical), and dh_tree_last_page_len is each
    node's token count mod 16."""
    rng = np.random.default_rng(13)
    pool = Pool(backend, 96, HKV, D, _lib.KV_BF16)
    mirror = Mirror(pool)
    tree = TreeState(KvCache(KvCacheConfig(num_kv_heads=HKV, head_dim=D, max_blocks=96)), 16)
    cfg = AttentionConfig(HQ, HKV, D)
    dec = TreeDecoder(backend, pool, tree, cfg, [NodeId.ROOT])
    def append(i):
        before = tree.get_block_table(dec.leaves[i]) or []
        page, off = dec.append_token(i, 2)
        after = tree.get_block_table(dec.leaves[i])
        if before and len(after) == len(before) and after[-1] != before[-1]:   # copy on write
            mirror.copy(int(before[-1]), int(after[-1]))
        mirror.write(page, off, rng)

    for _ in range(40):
        append(0)
    for _ in range(3):
        dec.fork(0)
    for i in range(1, 4):
        for _ in range(5 * i + 7):
            append(i)
    lpl = dec.last_page_len()
    assert list(lpl) == [tree.get_node(n).num_tokens % 16 for n in dec.leaves]
    q = _q(rng, len(dec.leaves))
    from dendrite_amd.backend import DecodePlan as DP
    a = _decode(DP.from_tree(backend, cfg, pool, tree, dec.leaves), q, lpl)
    b = _decode(_pages_plan(backend, pool, cfg, dec.tables()), q, lpl)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = _oracle(mirror, cfg, q, dec.tables(), lpl)
    assert excess_err(a, ref, _lib.DTYPE_BF16) <= TOL[_lib.DTYPE_BF16]
