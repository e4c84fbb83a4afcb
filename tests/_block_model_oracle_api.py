"""The block-model API of dendrite_amd.cache (BlockTable, BlockPool, KvCache,
TreeState, BlockId, NodeId) implemented over the test oracle's pure-Python
restatement (oracle/block_model.py), so the reference's ported integer tests
in test_block_model.py run, unchanged, against the oracle as well as against
the C++ product.  Errors surface as OracleError, which those tests see under
the name DhError.  Test infrastructure only."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from oracle import block_model as ref


class OracleError(RuntimeError):
    pass


class BlockId(int):
    INVALID: "BlockId"

    def is_valid(self) -> bool:
        return int(self) != ref.INVALID


BlockId.INVALID = BlockId(ref.INVALID)


class NodeId(int):
    ROOT: "NodeId"
    INVALID: "NodeId"

    def is_valid(self) -> bool:
        return int(self) != 0xFFFFFFFFFFFFFFFF


NodeId.ROOT = NodeId(0)
NodeId.INVALID = NodeId(0xFFFFFFFFFFFFFFFF)


def _call(fn, *args):
    try:
        return fn(*args)
    except (ref.OutOfMemory, ref.InvalidBlock, ref.InvalidNode) as e:
        raise OracleError(repr(e)) from None


class BlockTable:
    def __init__(self, tokens_per_block: int = 16, _table: Optional[ref.BlockTable] = None):
        self._t = _table if _table is not None else ref.BlockTable(tokens_per_block)
        self.tokens_per_block = tokens_per_block

    @classmethod
    def new(cls, tokens_per_block: int = 16) -> "BlockTable":
        return cls(tokens_per_block)

    @classmethod
    def with_capacity(cls, tokens_per_block: int, max_blocks: int) -> "BlockTable":
        return cls(tokens_per_block)

    def num_blocks(self) -> int:
        return len(self._t.blocks)

    def num_tokens(self) -> int:
        return self._t.num_tokens

    def get(self, i: int) -> Optional[BlockId]:
        b = self._t.get(i)
        return None if b is None else BlockId(b)

    def block_for_token(self, pos: int) -> Optional[BlockId]:
        b = self._t.block_for_token(pos)
        return None if b is None else BlockId(b)

    def push(self, b: int) -> None:
        self._t.push(int(b))

    def set(self, i: int, b: int) -> None:
        self._t.set(i, int(b))

    def set_num_tokens(self, n: int) -> None:
        self._t.num_tokens = n

    def add_tokens(self, n: int) -> None:
        self._t.num_tokens += n

    def blocks(self) -> list[BlockId]:
        return [BlockId(b) for b in self._t.blocks]

    def needs_new_block(self) -> bool:
        return self._t.needs_new_block()

    def fork(self) -> "BlockTable":
        return BlockTable(self.tokens_per_block, _table=self._t.fork())

    def clear(self) -> None:
        self._t.blocks.clear()
        self._t.num_tokens = 0


class BlockPool:
    def __init__(self, max_blocks: int, tokens_per_block: int = 16):
        self._p = ref.BlockPool(max_blocks, tokens_per_block)
        self.tokens_per_block = tokens_per_block

    def allocate(self) -> BlockId:
        return BlockId(_call(self._p.allocate))

    def free(self, b: int) -> None:
        _call(self._p.free, int(b))

    def share(self, b: int) -> None:
        _call(self._p.share, int(b))

    def copy_on_write(self, b: int) -> BlockId:
        return BlockId(_call(self._p.copy_on_write, int(b)))

    def free_count(self) -> int:
        return self._p.free_count()

    def total(self) -> int:
        return len(self._p.refcount)

    def get_refcount(self, b: int) -> Optional[int]:
        return self._p.refcount[int(b)] if 0 <= int(b) < self.total() else None


@dataclass
class KvCacheConfig:
    num_layers: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    max_blocks: int = 65536
    tokens_per_block: int = 16


class KvCache:
    def __init__(self, config: KvCacheConfig):
        self._config = config
        self.pool = BlockPool(config.max_blocks, config.tokens_per_block)

    def config(self) -> KvCacheConfig:
        return self._config

    def allocate_block(self) -> BlockId:
        return self.pool.allocate()

    def free_block(self, b: int) -> None:
        self.pool.free(b)

    def share_block(self, b: int) -> None:
        self.pool.share(b)

    def copy_on_write(self, b: int) -> BlockId:
        return self.pool.copy_on_write(b)

    def free_blocks(self) -> int:
        return self.pool.free_count()

    def total_blocks(self) -> int:
        return self._config.max_blocks

    def used_blocks(self) -> int:
        return self._config.max_blocks - self.pool.free_count()


@dataclass
class ForkHandle:
    node_id: NodeId
    depth: int
    num_tokens: int


@dataclass
class NodeInfo:
    id: NodeId
    parent: Optional[NodeId]
    num_tokens: int
    num_children: int
    is_active: bool


class TreeState:
    def __init__(self, kv_cache: KvCache, tokens_per_block: int = 16):
        self.kv_cache = kv_cache
        self._s = ref.TreeState(kv_cache.pool._p, tokens_per_block)

    def fork(self, frm: int) -> ForkHandle:
        nid, depth, ntok = _call(self._s.fork, int(frm))
        return ForkHandle(NodeId(nid), depth, ntok)

    def append_token(self, nid: int, token: int):
        cow = _call(self._s.append_token, int(nid), int(token))
        return None if cow is None else (BlockId(cow[0]), BlockId(cow[1]))

    def release(self, nid: int) -> None:
        _call(self._s.release, int(nid))

    def get_node(self, nid: int) -> Optional[NodeInfo]:
        n = self._s.nodes.get(int(nid))
        if n is None:
            return None
        return NodeInfo(NodeId(n.id), None if n.parent is None else NodeId(n.parent), n.table.num_tokens,
                        n.num_children, n.active)

    def get_block_table(self, nid: int) -> Optional[list[BlockId]]:
        n = self._s.nodes.get(int(nid))
        return None if n is None else [BlockId(b) for b in n.table.blocks]

    def get_tokens(self, nid: int) -> Optional[list[int]]:
        n = self._s.nodes.get(int(nid))
        return None if n is None else list(n.tokens)

    def num_nodes(self) -> int:
        return len(self._s.nodes)

    @property
    def tokens_per_block(self) -> int:
        return self._s.nodes[0].table.tokens_per_block
