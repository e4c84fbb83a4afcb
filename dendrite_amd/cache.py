"""Host block model over the C ABI, with the names of Dendrite's cache/tree API.

  BlockId, BlockPool, KvCache, KvCacheConfig   crates/dendrite-core/src/cache/
                                               {block.rs, pool.rs, mod.rs}
  BlockTable                                   cache/block_table.rs
  TreeState, NodeId, ForkHandle, NodeInfo      crates/dendrite-core/src/tree/
                                               {state.rs, node.rs}
The implementation is the C++ block model inside libdendrite_hip.so.
"""
from __future__ import annotations

import ctypes as C
import itertools
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import DhError, check, lib


class BlockId(int):
    """u32 physical block id; INVALID = u32::MAX (cache/block.rs:7-16)."""

    INVALID: "BlockId"

    def is_valid(self) -> bool:
        return int(self) != _lib.INVALID_PAGE

    def __repr__(self) -> str:
        return f"BlockId({int(self)})"


BlockId.INVALID = BlockId(_lib.INVALID_PAGE)


class NodeId(int):
    """u64 tree node id; ROOT = 0, INVALID = u64::MAX (tree/node.rs:7-21)."""

    ROOT: "NodeId"
    INVALID: "NodeId"

    def is_valid(self) -> bool:
        return int(self) != _lib.INVALID_NODE

    def __repr__(self) -> str:
        return f"NodeId({int(self)})"


NodeId.ROOT = NodeId(_lib.ROOT_NODE)
NodeId.INVALID = NodeId(_lib.INVALID_NODE)


_table_uids = itertools.count(1)
# Bumped by every change of any table's block list (a cheap "did anything
# change" check before looking at each table's version).
_mutations = [0]


def block_table_mutations() -> int:
    return _mutations[0]


class BlockTable:
    """Logical -> physical block mapping of one sequence.

    uid (unique per object for the process) and version (bumped by every
    change of the block list: push, set, clear) let a caller cache what it
    derived from the list, e.g. HipBackend's decode plans; neither exists in
    the reference, whose decode re-reads every table on every call."""

    def __init__(self, tokens_per_block: int = 16, _handle=None):
        self._h = C.c_void_p()
        self._destroy = lib().dh_block_table_destroy
        if _handle is not None:
            self._h = _handle
        else:
            check(lib().dh_block_table_create(tokens_per_block, C.byref(self._h)))
        self.tokens_per_block = tokens_per_block
        self.uid = next(_table_uids)
        self.version = 0

    @classmethod
    def new(cls, tokens_per_block: int = 16) -> "BlockTable":
        return cls(tokens_per_block)

    @classmethod
    def with_capacity(cls, tokens_per_block: int, max_blocks: int) -> "BlockTable":
        return cls(tokens_per_block)

    def __del__(self):
        destroy = getattr(self, "_destroy", None)  # bound at construction
        if destroy is not None and getattr(self, "_h", None) and self._h.value:
            destroy(self._h)
            self._h = None

    def num_blocks(self) -> int:
        return lib().dh_block_table_num_blocks(self._h)

    def num_tokens(self) -> int:
        return lib().dh_block_table_num_tokens(self._h)

    def get(self, logical_idx: int) -> Optional[BlockId]:
        if logical_idx < 0:
            return None
        out = C.c_uint32()
        if lib().dh_block_table_get(self._h, logical_idx, C.byref(out)) != _lib.DH_OK:
            return None
        return BlockId(out.value)

    def block_for_token(self, token_pos: int) -> Optional[BlockId]:
        return self.get(token_pos // self.tokens_per_block)

    def push(self, block_id: int) -> None:
        check(lib().dh_block_table_push(self._h, int(block_id)))
        self.version += 1
        _mutations[0] += 1

    def set(self, logical_idx: int, block_id: int) -> None:
        check(lib().dh_block_table_set(self._h, logical_idx, int(block_id)))
        self.version += 1
        _mutations[0] += 1

    def set_num_tokens(self, count: int) -> None:
        check(lib().dh_block_table_set_num_tokens(self._h, count))

    def add_tokens(self, count: int) -> None:
        check(lib().dh_block_table_add_tokens(self._h, count))

    def blocks(self) -> list[BlockId]:
        n = lib().dh_block_table_blocks(self._h, None, 0)
        buf = (C.c_uint32 * max(1, n))()
        lib().dh_block_table_blocks(self._h, buf, n)
        return [BlockId(buf[i]) for i in range(n)]

    def block_ids(self) -> np.ndarray:
        """blocks() as a uint32 array (one copy out of the C model)."""
        n = lib().dh_block_table_blocks(self._h, None, 0)
        out = np.empty(n, dtype=np.uint32)
        if n:
            lib().dh_block_table_blocks(self._h, out.ctypes.data_as(_lib._PU32), n)
        return out

    def needs_new_block(self) -> bool:
        return bool(lib().dh_block_table_needs_new_block(self._h))

    def fork(self) -> "BlockTable":
        h = C.c_void_p()
        check(lib().dh_block_table_fork(self._h, C.byref(h)))
        return BlockTable(self.tokens_per_block, _handle=h)

    def clear(self) -> None:
        check(lib().dh_block_table_clear(self._h))
        self.version += 1
        _mutations[0] += 1

    @classmethod
    def from_blocks(cls, ids, num_tokens: Optional[int] = None, tokens_per_block: int = 16):
        t = cls(tokens_per_block)
        for b in ids:
            t.push(b)
        t.set_num_tokens(len(list(ids)) * tokens_per_block if num_tokens is None else num_tokens)
        return t


class BlockPool:
    """Refcounted block pool with a FIFO free list (cache/pool.rs)."""

    def __init__(self, max_blocks: int, tokens_per_block: int = 16):
        self._h = C.c_void_p()
        self._destroy = lib().dh_block_pool_destroy
        check(lib().dh_block_pool_create(max_blocks, tokens_per_block, C.byref(self._h)))
        self.tokens_per_block = tokens_per_block

    def __del__(self):
        destroy = getattr(self, "_destroy", None)  # bound at construction
        if destroy is not None and getattr(self, "_h", None) and self._h.value:
            destroy(self._h)
            self._h = None

    def allocate(self) -> BlockId:
        out = C.c_uint32()
        check(lib().dh_block_pool_allocate(self._h, C.byref(out)))
        return BlockId(out.value)

    def free(self, block_id: int) -> None:
        check(lib().dh_block_pool_free(self._h, int(block_id)))

    def share(self, block_id: int) -> None:
        check(lib().dh_block_pool_share(self._h, int(block_id)))

    def copy_on_write(self, block_id: int) -> BlockId:
        out = C.c_uint32()
        check(lib().dh_block_pool_copy_on_write(self._h, int(block_id), C.byref(out)))
        return BlockId(out.value)

    def free_count(self) -> int:
        return lib().dh_block_pool_free_count(self._h)

    def total(self) -> int:
        return lib().dh_block_pool_total(self._h)

    def get_refcount(self, block_id: int) -> Optional[int]:
        if not (0 <= int(block_id) < self.total()):
            return None
        return lib().dh_block_pool_refcount(self._h, int(block_id))


@dataclass
class KvCacheConfig:
    """cache/mod.rs:63-88."""

    num_layers: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    max_blocks: int = 65536
    tokens_per_block: int = 16


class KvCache:
    """cache/mod.rs:90-143: the block pool behind a config."""

    def __init__(self, config: KvCacheConfig):
        self._config = config
        self.pool = BlockPool(config.max_blocks, config.tokens_per_block)

    def config(self) -> KvCacheConfig:
        return self._config

    def allocate_block(self) -> BlockId:
        return self.pool.allocate()

    def free_block(self, block_id: int) -> None:
        self.pool.free(block_id)

    def share_block(self, block_id: int) -> None:
        self.pool.share(block_id)

    def copy_on_write(self, block_id: int) -> BlockId:
        return self.pool.copy_on_write(block_id)

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
    """Tree of CoW branches over a KvCache (tree/state.rs)."""

    def __init__(self, kv_cache: KvCache, tokens_per_block: int = 16):
        self.kv_cache = kv_cache          # keeps the pool alive
        self._h = C.c_void_p()
        self._destroy = lib().dh_tree_destroy
        check(lib().dh_tree_create(kv_cache.pool._h, tokens_per_block, C.byref(self._h)))

    def __del__(self):
        destroy = getattr(self, "_destroy", None)  # bound at construction
        if destroy is not None and getattr(self, "_h", None) and self._h.value:
            destroy(self._h)
            self._h = None

    def fork(self, from_node: int) -> ForkHandle:
        child, depth, ntok = C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(lib().dh_tree_fork(self._h, int(from_node), C.byref(child), C.byref(depth), C.byref(ntok)))
        return ForkHandle(NodeId(child.value), depth.value, ntok.value)

    def append_token(self, node_id: int, token: int):
        """Returns (old_block, new_block) when the append copied-on-write the
        node's last block, else None."""
        src, dst = C.c_uint32(), C.c_uint32()
        check(lib().dh_tree_append_token(self._h, int(node_id), int(token), C.byref(src), C.byref(dst)))
        if src.value == _lib.INVALID_PAGE:
            return None
        return BlockId(src.value), BlockId(dst.value)

    def release(self, node_id: int) -> None:
        check(lib().dh_tree_release(self._h, int(node_id)))

    def get_node(self, node_id: int) -> Optional[NodeInfo]:
        info = _lib.dh_node_info()
        if lib().dh_tree_get_node(self._h, int(node_id), C.byref(info)) != _lib.DH_OK:
            return None
        parent = None if info.parent == _lib.INVALID_NODE else NodeId(info.parent)
        return NodeInfo(NodeId(info.id), parent, info.num_tokens, info.num_children, bool(info.is_active))

    def get_block_table(self, node_id: int) -> Optional[list[BlockId]]:
        n = C.c_uint32()
        if lib().dh_tree_get_block_table(self._h, int(node_id), None, 0, C.byref(n)) != _lib.DH_OK:
            return None
        buf = (C.c_uint32 * max(1, n.value))()
        check(lib().dh_tree_get_block_table(self._h, int(node_id), buf, n.value, C.byref(n)))
        return [BlockId(buf[i]) for i in range(n.value)]

    def get_tokens(self, node_id: int) -> Optional[list[int]]:
        n = C.c_uint32()
        if lib().dh_tree_get_tokens(self._h, int(node_id), None, 0, C.byref(n)) != _lib.DH_OK:
            return None
        buf = (C.c_uint32 * max(1, n.value))()
        check(lib().dh_tree_get_tokens(self._h, int(node_id), buf, n.value, C.byref(n)))
        return [buf[i] for i in range(n.value)]

    def num_nodes(self) -> int:
        return lib().dh_tree_num_nodes(self._h)

    @property
    def tokens_per_block(self) -> int:
        return lib().dh_tree_tokens_per_block(self._h)


__all__ = ["BlockId", "NodeId", "BlockTable", "BlockPool", "KvCacheConfig", "KvCache",
           "ForkHandle", "NodeInfo", "TreeState", "DhError"]
