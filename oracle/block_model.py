"""TEST INFRASTRUCTURE ONLY: pure-Python restatement of Dendrite's block model,
used as the checker in differential tests of the C++ block model.

  BlockPool   crates/dendrite-core/src/cache/pool.rs:20-107
  BlockTable  crates/dendrite-core/src/cache/block_table.rs:19-109
  TreeState   crates/dendrite-core/src/tree/state.rs:33-197 (+ node.rs:58-146)

One deliberate difference from the Rust code, mirrored from the product: a
free of a block that is not allocated is an InvalidBlock error here (the
reference would decrement a free block's refcount of 1 and queue it twice).
"""
from __future__ import annotations

from collections import deque

INVALID = 0xFFFFFFFF


class OutOfMemory(Exception):
    pass


class InvalidBlock(Exception):
    pass


class InvalidNode(Exception):
    pass


class BlockPool:
    def __init__(self, max_blocks: int, tokens_per_block: int = 16):
        self.refcount = [0] * max_blocks
        self.free_list = deque(range(max_blocks))          # pool.rs:26-30
        self.tokens_per_block = tokens_per_block

    def allocate(self) -> int:                             # pool.rs:40-45
        if not self.free_list:
            raise OutOfMemory("no free blocks")
        b = self.free_list.popleft()
        self.refcount[b] = 1
        return b

    def _valid(self, b: int) -> bool:                      # pool.rs:105-107
        return 0 <= b < len(self.refcount)

    def free(self, b: int) -> None:                        # pool.rs:48-63
        if not self._valid(b) or self.refcount[b] == 0:
            raise InvalidBlock(b)
        self.refcount[b] -= 1
        if self.refcount[b] == 0:
            self.free_list.append(b)

    def share(self, b: int) -> None:                       # pool.rs:66-73
        if not self._valid(b):
            raise InvalidBlock(b)
        self.refcount[b] += 1

    def copy_on_write(self, b: int) -> int:                # pool.rs:76-97
        if not self._valid(b):
            raise InvalidBlock(b)
        if self.refcount[b] <= 1:
            return b
        nb = self.allocate()
        self.free(b)
        return nb

    def free_count(self) -> int:
        return len(self.free_list)


class BlockTable:
    def __init__(self, tokens_per_block: int = 16):
        self.blocks: list[int] = []
        self.num_tokens = 0
        self.tokens_per_block = tokens_per_block

    def get(self, i: int):                                 # block_table.rs:49-51
        return self.blocks[i] if 0 <= i < len(self.blocks) else None

    def block_for_token(self, pos: int):                   # block_table.rs:54-57
        return self.get(pos // self.tokens_per_block)

    def push(self, b: int) -> None:
        self.blocks.append(b)

    def set(self, i: int, b: int) -> None:                 # block_table.rs:65-70
        if i >= len(self.blocks):
            self.blocks.extend([INVALID] * (i + 1 - len(self.blocks)))
        self.blocks[i] = b

    def needs_new_block(self) -> bool:                     # block_table.rs:88-94
        if not self.blocks:
            return True
        return self.num_tokens % self.tokens_per_block == 0 and self.num_tokens > 0

    def fork(self) -> "BlockTable":                        # block_table.rs:97-103
        t = BlockTable(self.tokens_per_block)
        t.blocks = list(self.blocks)
        t.num_tokens = self.num_tokens
        return t


class _Node:
    def __init__(self, nid, parent, table):
        self.id, self.parent, self.table = nid, parent, table
        self.tokens: list[int] = []
        self.num_children = 0
        self.active = True


class TreeState:
    ROOT = 0

    def __init__(self, pool: BlockPool, tokens_per_block: int = 16):
        self.pool = pool
        self.next_id = 1
        self.nodes = {0: _Node(0, None, BlockTable(tokens_per_block))}

    def fork(self, frm: int):                              # state.rs:49-84
        if frm not in self.nodes:
            raise InvalidNode(frm)
        parent = self.nodes[frm]
        child = _Node(self.next_id, frm, parent.table.fork())
        self.next_id += 1
        for b in child.table.blocks:
            if b != INVALID:
                self.pool.share(b)
        parent.num_children += 1
        # state.rs:157-171: the walk stops at a parent that was collected
        # (a released node with no children left, whose child lives on).
        depth, cur = 0, frm
        while cur in self.nodes and self.nodes[cur].parent is not None:
            depth += 1
            cur = self.nodes[cur].parent
        self.nodes[child.id] = child
        return child.id, depth + 1, child.table.num_tokens

    def append_token(self, nid: int, token: int):          # state.rs:87-113
        if nid not in self.nodes:
            raise InvalidNode(nid)
        node = self.nodes[nid]
        cow = None
        if node.table.needs_new_block():
            node.table.push(self.pool.allocate())
        if node.table.blocks:
            last = node.table.blocks[-1]
            nb = self.pool.copy_on_write(last)
            if nb != last:
                node.table.blocks[-1] = nb
                cow = (last, nb)
        node.tokens.append(token)
        node.table.num_tokens += 1
        return cow

    def release(self, nid: int) -> None:                   # state.rs:116-134, 174-196
        node = self.nodes.get(nid)
        if node is not None:
            node.active = False
            if node.parent is not None and node.parent in self.nodes:
                p = self.nodes[node.parent]
                p.num_children = max(0, p.num_children - 1)
        victims = [i for i, n in self.nodes.items() if i != 0 and not n.active and n.num_children == 0]
        for i in victims:
            for b in self.nodes[i].table.blocks:
                if b != INVALID:
                    self.pool.free(b)
            del self.nodes[i]
