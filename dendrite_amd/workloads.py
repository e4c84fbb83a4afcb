"""Seeded synthetic decode workloads: the five configurations of the benchmark.

  c1  TinyLlama-shape single sequence, f32, 512 tokens in 32 pages, 32/4/64.
  c2  TinyLlama-shape fork: 6 branches share a 4096-token prefix (256 pages,
      refcount 6), each with a private 256-token suffix on shuffled pages; bf16.
  c3  Llama-3-8B-shape MCTS tree: 8192-token root, 3 levels of fan-out 4 adding
      128 tokens each (64 leaves), pages shuffled over a 65536-page pool; bf16,
      32/8/128.  The headline workload.
  c4  Llama-3-8B-shape FP8 E4M3 KV (fp32 scale per page/head/plane): 256
      sequences with T ~ U[512, 4096], every 8th forked from its predecessor at
      a random block boundary.
  c5  Llama-3-70B one-GPU-share with MXFP8 KV: 32 requests x 32768-token shared
      prefix, 16 beams each (512 leaves) with 512-token private suffixes;
      64/8/128, 1% outliers at 20 sigma.

Tree shapes follow what TreeState::fork/append_token produce
(crates/dendrite-core/src/tree/state.rs:49-113): a child's table is the
parent's table (shared pages, refcount + 1) followed by its own pages.
K/V/q values come from dh_synth_* (SplitMix64 + Box-Muller) in
libdendrite_testdata.so, so a page's content depends only on (seed, page id).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import _lib
from ._lib import check_testdata, testdata_lib

_KV_EB = {_lib.KV_F16: 2, _lib.KV_BF16: 2, _lib.KV_F32: 4, _lib.KV_FP8_E4M3: 1, _lib.KV_MXFP8: 1}
_Q_EB = {_lib.DTYPE_F16: 2, _lib.DTYPE_BF16: 2, _lib.DTYPE_F32: 4}


@dataclass
class Workload:
    name: str
    hq: int
    hkv: int
    d: int
    q_dtype: int
    kv_format: int
    num_pool_pages: int
    indptr: np.ndarray
    indices: np.ndarray
    last_page_len: np.ndarray
    seed: int
    outlier: float = 0.0
    outlier_every: int = 0
    gqa_mapping: int = _lib.GQA_TILED
    description: str = ""
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return len(self.indptr) - 1

    @property
    def page_bytes(self) -> int:
        return 2 * self.hkv * 16 * self.d * _KV_EB[self.kv_format]

    @property
    def scale_bytes(self) -> int:
        if self.kv_format == _lib.KV_FP8_E4M3:
            return 2 * self.hkv * 4
        if self.kv_format == _lib.KV_MXFP8:
            return 2 * self.hkv * 16 * (self.d // 32)
        return 0

    def seq_pages(self, b: int) -> np.ndarray:
        return self.indices[self.indptr[b]:self.indptr[b + 1]]

    def seq_len(self, b: int) -> int:
        n = int(self.indptr[b + 1] - self.indptr[b])
        if n == 0:
            return 0
        lp = int(self.last_page_len[b])
        return 16 * (n - 1) + (16 if lp <= 0 or lp > 16 else lp)

    def page_ids(self) -> np.ndarray:
        ids = self.indices[self.indices != _lib.INVALID_PAGE]
        return np.unique(ids).astype(np.uint32)

    def make_pages(self, ids: Optional[np.ndarray] = None):
        """Host page records for `ids` (default all referenced pages):
        (data uint8 [n, page_bytes], scales uint8 [n, scale_bytes] or None)."""
        ids = self.page_ids() if ids is None else np.ascontiguousarray(ids, dtype=np.uint32)
        data = np.empty((len(ids), self.page_bytes), dtype=np.uint8)
        scales = np.empty((len(ids), self.scale_bytes), dtype=np.uint8) if self.scale_bytes else None
        check_testdata(testdata_lib().dh_synth_pages(self.kv_format, self.hkv, self.d, self.seed,
                                   ids.ctypes.data_as(_lib._PU32), len(ids), float(self.outlier),
                                   self.outlier_every, data.ctypes.data_as(C.c_void_p),
                                   None if scales is None else scales.ctypes.data_as(C.c_void_p)))
        return data, scales

    def make_q(self) -> np.ndarray:
        """Raw query bits [B][Hq][D] (uint16 for f16/bf16, float32 for f32)."""
        n = self.batch * self.hq * self.d
        dt = np.float32 if self.q_dtype == _lib.DTYPE_F32 else np.uint16
        q = np.empty(n, dtype=dt)
        check_testdata(testdata_lib().dh_synth_fill(q.ctypes.data_as(C.c_void_p), self.q_dtype, self.seed ^ 0x51,
                                  0, n))
        return q.reshape(self.batch, self.hq, self.d)

    def attention_config(self):
        from .backend import AttentionConfig
        cfg = AttentionConfig(self.hq, self.hkv, self.d)
        cfg.q_dtype = self.q_dtype
        cfg.kv_format = self.kv_format
        cfg.gqa_mapping = self.gqa_mapping
        return cfg

    # --- accounting (algorithmic bytes / flops per step) ------------------
    def page_valid_tokens(self) -> dict:
        """Valid tokens of each referenced page (the most any sequence reads)."""
        valid: dict[int, int] = {}
        for b in range(self.batch):
            pl = [int(p) for p in self.seq_pages(b) if p != _lib.INVALID_PAGE]
            for i, p in enumerate(pl):
                n = 16
                if i == len(pl) - 1:
                    lp = int(self.last_page_len[b])
                    n = 16 if lp <= 0 or lp > 16 else lp
                valid[p] = max(valid.get(p, 0), n)
        return valid

    def algorithmic_bytes(self) -> int:
        """Unique KV bytes (valid tokens of each referenced page, once, plus
        scale bytes) + Q + O."""
        eb = _KV_EB[self.kv_format]
        tok_bytes = 2 * self.hkv * self.d * eb
        total = 0
        for n in self.page_valid_tokens().values():
            total += n * tok_bytes
            if self.kv_format == _lib.KV_FP8_E4M3:
                total += 2 * self.hkv * 4
            elif self.kv_format == _lib.KV_MXFP8:
                total += n * 2 * self.hkv * (self.d // 32)
        qo = 2 * self.batch * self.hq * self.d * _Q_EB[self.q_dtype]
        return total + qo

    def flops(self) -> int:
        return 4 * self.hq * self.d * sum(self.seq_len(b) for b in range(self.batch))

    def naive_kv_bytes(self) -> int:
        """KV bytes if every sequence re-read its pages (no sharing)."""
        return sum(self.seq_len(b) for b in range(self.batch)) * 2 * self.hkv * self.d * _KV_EB[self.kv_format]


def _csr(tables, lpl=None):
    indptr = np.zeros(len(tables) + 1, dtype=np.uint32)
    for i, t in enumerate(tables):
        indptr[i + 1] = indptr[i] + len(t)
    indices = np.concatenate([np.asarray(t, dtype=np.uint32) for t in tables]) if tables else \
        np.zeros(0, dtype=np.uint32)
    if lpl is None:
        lpl = np.full(len(tables), 16, dtype=np.int32)
    return indptr, indices.astype(np.uint32), np.asarray(lpl, dtype=np.int32)


def c1(seed: int = 0xC1) -> Workload:
    tables = [list(range(32))]
    ip, ix, lp = _csr(tables)
    return Workload("c1", 32, 4, 64, _lib.DTYPE_F32, _lib.KV_F32, 32, ip, ix, lp, seed,
                    description="TinyLlama single sequence, f32, 512 tokens / 32 pages, 32/4/64")


def c2(seed: int = 0xC2, branches: int = 6, prefix_pages: int = 256, suffix_pages: int = 16,
       pool_pages: int = 1024) -> Workload:
    perm = np.random.Generator(np.random.PCG64(seed)).permutation(pool_pages).astype(np.uint32)
    prefix = list(perm[:prefix_pages])
    tables = []
    for i in range(branches):
        s = prefix_pages + i * suffix_pages
        tables.append(prefix + list(perm[s:s + suffix_pages]))
    ip, ix, lp = _csr(tables)
    return Workload("c2", 32, 4, 64, _lib.DTYPE_BF16, _lib.KV_BF16, pool_pages, ip, ix, lp, seed,
                    description=f"TinyLlama fork, bf16, {branches} branches x ({prefix_pages * 16} shared"
                                f" + {suffix_pages * 16} private tokens), 32/4/64")


def tree_tables(root_pages: int, fanout: int, levels: int, level_pages: int, page_src):
    """Leaf tables of a tree: root run, then one run per level node."""
    it = iter(page_src)
    root = [next(it) for _ in range(root_pages)]
    frontier = [root]
    for _ in range(levels):
        nxt = []
        for parent in frontier:
            for _ in range(fanout):
                nxt.append(parent + [next(it) for _ in range(level_pages)])
        frontier = nxt
    return frontier


def c3(seed: int = 0xC3, rotation: int = 0, root_pages: int = 512, fanout: int = 4, levels: int = 3,
       level_pages: int = 8, pool_pages: int = 65536) -> Workload:
    """rotation k uses the k-th disjoint run of the shuffled pool, so several
    rotations have disjoint working sets (used to defeat the last-level cache
    when timing)."""
    perm = np.random.Generator(np.random.PCG64(seed)).permutation(pool_pages).astype(np.uint32)
    n_nodes = sum(fanout ** l for l in range(1, levels + 1))
    per_tree = root_pages + n_nodes * level_pages
    if (rotation + 1) * per_tree > pool_pages:
        raise ValueError("rotation does not fit the pool")
    src = [int(x) for x in perm[rotation * per_tree:(rotation + 1) * per_tree]]
    tables = tree_tables(root_pages, fanout, levels, level_pages, src)
    ip, ix, lp = _csr(tables)
    return Workload("c3", 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, pool_pages, ip, ix, lp, seed,
                    description=f"Llama-3-8B MCTS tree, bf16, {root_pages * 16}-token root + {levels} levels"
                                f" x fan-out {fanout} x {level_pages * 16} tokens ({len(tables)} leaves), "
                                "32/8/128",
                    meta={"rotation": rotation, "pages_per_tree": per_tree})


def c4(seed: int = 0xC4, n_seqs: int = 256, tmin: int = 512, tmax: int = 4096,
       pool_pages: int = 65536, fork_every: int = 8) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    perm = rng.permutation(pool_pages).astype(np.uint32)
    nxt = 0
    tables, lpl = [], []
    for i in range(n_seqs):
        T = int(rng.integers(tmin, tmax + 1))
        n = (T + 15) // 16
        lp = T - 16 * (n - 1)
        if i % fork_every == fork_every - 1 and i > 0:
            prev = tables[-1]
            b = int(rng.integers(1, min(len(prev), n) - 1 + 1))
            t = list(prev[:b]) + [int(x) for x in perm[nxt:nxt + n - b]]
            nxt += n - b
        else:
            t = [int(x) for x in perm[nxt:nxt + n]]
            nxt += n
        tables.append(t)
        lpl.append(lp)
    ip, ix, lp = _csr(tables, lpl)
    return Workload("c4", 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_FP8_E4M3, pool_pages, ip, ix, lp, seed,
                    description=f"Llama-3-8B FP8-E4M3 KV, {n_seqs} sequences T~U[{tmin},{tmax}], every "
                                f"{fork_every}th forked, 32/8/128")


def c5(seed: int = 0xC5, requests: int = 32, prefix_pages: int = 2048, beams: int = 16,
       suffix_pages: int = 32, pool_pages: Optional[int] = None, outlier: float = 20.0,
       outlier_every: int = 100) -> Workload:
    need = requests * prefix_pages + requests * beams * suffix_pages
    pool_pages = pool_pages or max(need, 98304)
    perm = np.random.Generator(np.random.PCG64(seed)).permutation(pool_pages).astype(np.uint32)
    nxt = 0
    tables = []
    for _ in range(requests):
        prefix = [int(x) for x in perm[nxt:nxt + prefix_pages]]
        nxt += prefix_pages
        for _ in range(beams):
            tables.append(prefix + [int(x) for x in perm[nxt:nxt + suffix_pages]])
            nxt += suffix_pages
    ip, ix, lp = _csr(tables)
    return Workload("c5", 64, 8, 128, _lib.DTYPE_BF16, _lib.KV_MXFP8, pool_pages, ip, ix, lp, seed,
                    outlier=outlier, outlier_every=outlier_every,
                    description=f"Llama-3-70B share, MXFP8 KV, {requests} x {prefix_pages * 16}-token prefix x"
                                f" {beams} beams + {suffix_pages * 16}-token suffixes, 64/8/128")


def custom(tables, hq: int, hkv: int, d: int, q_dtype: int, kv_format: int, pool_pages: int,
           last_page_len=None, seed: int = 0xD0, name: str = "custom", **kw) -> Workload:
    """Any head shape / format over explicit page tables."""
    ip, ix, lp = _csr([list(t) for t in tables], last_page_len)
    return Workload(name, hq, hkv, d, q_dtype, kv_format, pool_pages, ip, ix, lp, seed, **kw)


def random_tree(seed: int, hq: int, hkv: int, d: int, q_dtype: int, kv_format: int,
                n_leaves: int = 12, pool_pages: int = 2048, max_depth: int = 4, max_run: int = 9,
                partial: bool = True, **kw) -> Workload:
    """Random fork tree: each node adds 0..max_run pages to its parent's table;
    leaves optionally end on a partial page."""
    rng = np.random.Generator(np.random.PCG64(seed))
    perm = [int(x) for x in rng.permutation(pool_pages)]
    nxt = [0]

    def take(n):
        out = perm[nxt[0]:nxt[0] + n]
        nxt[0] += n
        return out

    tables = [take(int(rng.integers(0, max_run + 1)))]
    while len(tables) < n_leaves:
        parent = tables[int(rng.integers(0, len(tables)))]
        tables.append(parent + take(int(rng.integers(0, max_run + 1))))
        if rng.random() < 0.3 and len(tables[-1]) > 0:
            tables[-1] = tables[-1][:int(rng.integers(0, len(tables[-1]) + 1))]
    lpl = [int(rng.integers(1, 17)) if partial else 16 for _ in tables]
    return custom(tables, hq, hkv, d, q_dtype, kv_format, pool_pages, lpl, seed=seed,
                  name=f"tree{seed}", **kw)


def c3prefix(seed: int = 0xC3) -> Workload:
    """C3's shared-prefix stage alone: the 8192-token root shared by 64
    leaves, each with one private page (MFMA counters of the prefix kernel
    path without the tree's other levels)."""
    w = c3(seed, root_pages=512, fanout=64, levels=1, level_pages=1)
    w.name = "c3prefix"
    w.description = "C3 root alone: 8192-token prefix shared by 64 leaves + 1 private page each, bf16, 32/8/128"
    return w


ALL = {"c1": c1, "c2": c2, "c3": c3, "c4": c4, "c5": c5, "c3prefix": c3prefix}
