"""Python host side of the HIP decode path, over the C ABI.

  AttentionConfig  crates/dendrite-core/src/attention/backend.rs:17-59
  HipBackend       the AttentionBackend trait (backend.rs:61-97) for the
                   FlashInferBackend slot (attention/flashinfer.rs:211-269)
  Pool / DecodePlan / decode_batch
                   the raw C ABI (device page pool, decode plan, one step) that
                   replaces dendrite-ffi's BatchDecodeKernel / CascadeAttention
                   (crates/dendrite-ffi/src/flashinfer/{batch_decode,cascade}.rs)

torch is used only to hold device memory and streams.  Every computation runs
in libdendrite_hip.so; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import threading
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import DhError, check, lib
from .cache import BlockTable


def _torch():
    import torch  # noqa: PLC0415 — plumbing only, imported on first device use
    return torch


def dtype_code(t) -> int:
    torch = _torch()
    return {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16,
            torch.float32: _lib.DTYPE_F32}[t]


def torch_dtype(code: int):
    torch = _torch()
    return {_lib.DTYPE_F16: torch.float16, _lib.DTYPE_BF16: torch.bfloat16,
            _lib.DTYPE_F32: torch.float32}[code]


def raw_to_tensor(raw: np.ndarray, q_dtype: int, device: str = "cuda:0"):
    """Device tensor from raw host bits (uint16 for f16/bf16, float32)."""
    torch = _torch()
    raw = np.ascontiguousarray(raw)
    if q_dtype == _lib.DTYPE_F32:
        return torch.from_numpy(raw.view(np.float32)).to(device)
    t = torch.from_numpy(raw.view(np.int16))
    return t.view(torch.bfloat16 if q_dtype == _lib.DTYPE_BF16 else torch.float16).to(device)


def _as_torch_stream(stream):
    """torch stream object for a stream argument (None: the current stream;
    an int: a raw hipStream_t handle)."""
    torch = _torch()
    if stream is None:
        return torch.cuda.current_stream()
    if isinstance(stream, int):
        return torch.cuda.ExternalStream(stream)
    return stream


def _stream_ptr(stream) -> Optional[int]:
    """The hipStream_t of `stream` (a torch stream or a raw handle); None:
    torch's current stream on the current device (read through torch's raw
    accessor, which builds no Stream object, when this build has it)."""
    if stream is None:
        torch = _torch()
        raw, dev = getattr(torch._C, "_cuda_getCurrentRawStream", None), getattr(torch._C, "_cuda_getDevice", None)
        if raw is not None and dev is not None:
            return raw(dev())
        return torch.cuda.current_stream().cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


class AttentionConfig:
    """AttentionConfig (backend.rs:17-59) plus the GQA mapping and dtypes."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int):
        c = _lib.dh_attn_config()
        check(lib().dh_attn_config_init(C.byref(c), num_heads, num_kv_heads, head_dim))
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.scale = float(c.scale)               # 1/sqrt(head_dim) in f32 (backend.rs:37)
        self.sliding_window: Optional[int] = None
        self.gqa_mapping = _lib.GQA_TILED         # ReferenceBackend's Tensor::repeat
        self.q_dtype = _lib.DTYPE_BF16
        self.kv_format = _lib.KV_BF16

    @classmethod
    def new(cls, num_heads: int, num_kv_heads: int, head_dim: int) -> "AttentionConfig":
        return cls(num_heads, num_kv_heads, head_dim)

    @classmethod
    def default(cls) -> "AttentionConfig":        # backend.rs:54-58
        return cls(8, 8, 64)

    def with_sliding_window(self, window: int) -> "AttentionConfig":
        self.sliding_window = window
        return self

    def num_queries_per_kv(self) -> int:
        return self.num_heads // self.num_kv_heads

    def to_c(self) -> _lib.dh_attn_config:
        c = _lib.dh_attn_config()
        c.num_heads, c.num_kv_heads, c.head_dim = self.num_heads, self.num_kv_heads, self.head_dim
        c.scale = self.scale
        c.sliding_window = self.sliding_window or 0
        c.gqa_mapping = self.gqa_mapping
        c.q_dtype = self.q_dtype
        c.kv_format = self.kv_format
        return c


class Backend:
    """dh_backend: one HIP device."""

    def __init__(self, device: int = 0):
        self._h = C.c_void_p()
        self._destroy = lib().dh_destroy
        check(lib().dh_create(device, C.byref(self._h)))
        self.device = device

    def __del__(self):
        # Bound at construction: module globals may already be gone when an
        # object is collected at interpreter shutdown.
        destroy = getattr(self, "_destroy", None)
        if destroy is not None and getattr(self, "_h", None) and self._h.value:
            destroy(self._h)
            self._h = None

    def synchronize(self) -> None:
        check(lib().dh_synchronize(self._h))

    def memory_info(self) -> tuple[int, int]:
        f, t = C.c_size_t(), C.c_size_t()
        check(lib().dh_memory_info(self._h, C.byref(f), C.byref(t)))
        return f.value, t.value


def is_available() -> bool:
    return bool(lib().dh_is_available())


class Pool:
    """Device page pool [P][2][Hkv][16][D] (+ scale records)."""

    def __init__(self, backend: Backend, num_pages: int, num_kv_heads: int, head_dim: int,
                 kv_format: int = _lib.KV_BF16, page_size: int = _lib.PAGE_SIZE):
        self.backend = backend
        self._h = C.c_void_p()
        self._destroy = lib().dh_pool_destroy
        check(lib().dh_pool_create(backend._h, num_pages, num_kv_heads, head_dim, page_size,
                                   kv_format, C.byref(self._h)))
        self.num_pages = num_pages
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.kv_format = kv_format
        self.page_bytes = lib().dh_pool_page_bytes(self._h)
        self.scale_bytes = lib().dh_pool_scale_bytes(self._h)

    def __del__(self):
        # Bound at construction: module globals may already be gone when an
        # object is collected at interpreter shutdown.
        destroy = getattr(self, "_destroy", None)
        if destroy is not None and getattr(self, "_h", None) and self._h.value:
            destroy(self._h)
            self._h = None

    def write_pages(self, page_ids, data: np.ndarray, scales: Optional[np.ndarray] = None,
                    stream=None) -> None:
        ids = np.ascontiguousarray(page_ids, dtype=np.uint32)
        data = np.ascontiguousarray(data)
        assert data.nbytes == len(ids) * self.page_bytes, "data size does not match the pages"
        sp = None
        if self.scale_bytes:
            scales = np.ascontiguousarray(scales)
            assert scales.nbytes == len(ids) * self.scale_bytes, "scale size does not match the pages"
            sp = scales.ctypes.data_as(C.c_void_p)
        check(lib().dh_pool_write_pages(self._h, ids.ctypes.data_as(_lib._PU32), len(ids),
                                        data.ctypes.data_as(C.c_void_p), sp,
                                        _stream_ptr(stream) if stream is not None else None))

    def write_pages_device(self, page_ids, src, stream=None) -> None:
        """Quantise-on-write from device tensors: page_ids (uint32 / int32,
        [n]) receive src ([n, 2, num_kv_heads, 16, head_dim] float32 /
        bfloat16 / float16, K then V, zero past a partial page's tokens) in
        the pool's format (dh_pool_write_pages_device), on `stream` (default:
        torch's current stream).  Ids outside the pool are skipped."""
        torch = _torch()
        dtype = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16,
                 torch.float16: _lib.DTYPE_F16}.get(src.dtype)
        if dtype is None:
            raise DhError(_lib.DH_EINVAL, f"source dtype {src.dtype} (float32, bfloat16 or float16)")
        want = (2, self.num_kv_heads, _lib.PAGE_SIZE, self.head_dim)
        if src.dim() != 5 or tuple(src.shape[1:]) != want or src.shape[0] != page_ids.numel():
            raise DhError(_lib.DH_EINVAL, f"src shape {tuple(src.shape)} is not [n, *{want}]")
        if not (src.is_cuda and page_ids.is_cuda and src.is_contiguous() and page_ids.is_contiguous()):
            raise DhError(_lib.DH_EINVAL, "page_ids and src must be contiguous device tensors")
        if page_ids.dtype not in (torch.int32, torch.uint32):
            raise DhError(_lib.DH_EINVAL, "page_ids must be int32 or uint32")
        check(lib().dh_pool_write_pages_device(self._h, C.c_void_p(page_ids.data_ptr()), page_ids.numel(),
                                               C.c_void_p(src.data_ptr()), dtype, _stream_ptr(stream)))

    def write_tokens(self, page_id: int, tok_offset: int, k: np.ndarray, v: np.ndarray,
                     k_scale=None, v_scale=None, stream=None) -> None:
        """k, v: [num_kv_heads][n_tok][head_dim] in the pool's element format."""
        k = np.ascontiguousarray(k)
        v = np.ascontiguousarray(v)
        n_tok = k.shape[1]
        ks = None if k_scale is None else np.ascontiguousarray(k_scale)
        vs = None if v_scale is None else np.ascontiguousarray(v_scale)
        check(lib().dh_pool_write_tokens(self._h, page_id, tok_offset, n_tok,
                                         k.ctypes.data_as(C.c_void_p), v.ctypes.data_as(C.c_void_p),
                                         None if ks is None else ks.ctypes.data_as(C.c_void_p),
                                         None if vs is None else vs.ctypes.data_as(C.c_void_p),
                                         _stream_ptr(stream) if stream is not None else None))
        if stream is None:
            self.backend.synchronize()

    def copy_page(self, src: int, dst: int, stream=None) -> None:
        check(lib().dh_pool_copy_page(self._h, src, dst,
                                      _stream_ptr(stream) if stream is not None else None))

    def read_page(self, page_id: int) -> tuple[np.ndarray, Optional[np.ndarray]]:
        data = np.empty(self.page_bytes, dtype=np.uint8)
        scales = np.empty(self.scale_bytes, dtype=np.uint8) if self.scale_bytes else None
        check(lib().dh_pool_read_page(self._h, page_id, data.ctypes.data_as(C.c_void_p),
                                      None if scales is None else scales.ctypes.data_as(C.c_void_p)))
        return data, scales

    def gather(self, page_ids, kv_head: int):
        """dh_gather_debug: [2][n][16][D] raw bytes of the selected planes."""
        torch = _torch()
        ids = np.ascontiguousarray(page_ids, dtype=np.uint32)
        eb = self.page_bytes // (2 * self.num_kv_heads * 16 * self.head_dim)
        out = torch.empty(max(1, 2 * len(ids) * 16 * self.head_dim * eb), dtype=torch.uint8,
                          device=f"cuda:{self.backend.device}")
        n_out = C.c_uint32()
        check(lib().dh_gather_debug(self._h, ids.ctypes.data_as(_lib._PU32), len(ids), kv_head,
                                    C.c_void_p(out.data_ptr()), C.byref(n_out), None))
        n = n_out.value
        return out[: 2 * n * 16 * self.head_dim * eb].cpu().numpy(), n


class DecodePlan:
    """dh_plan: the work decomposition of one decode step."""

    def __init__(self, backend: Backend, config: AttentionConfig, pool: Pool, indptr, indices,
                 cascade: bool = True, shared_chunk_pages: int = 0, private_chunk_pages: int = 0,
                 target_items: int = 0, direct: bool = True):
        self.backend = backend
        self.pool = pool
        self.config = config
        ip = np.ascontiguousarray(indptr, dtype=np.uint32)
        ix = np.ascontiguousarray(indices, dtype=np.uint32)
        self.batch_size = len(ip) - 1
        opt = _lib.dh_plan_options()
        opt.shared_chunk_pages = shared_chunk_pages
        opt.private_chunk_pages = private_chunk_pages
        opt.target_items = target_items
        opt.direct = _lib.DIRECT_AUTO if direct else _lib.DIRECT_OFF
        self._c = config.to_c()
        self._h = C.c_void_p()
        self._destroy = lib().dh_plan_destroy
        check(lib().dh_plan_create(backend._h, C.byref(self._c), pool._h,
                                   ip.ctypes.data_as(_lib._PU32),
                                   ix.ctypes.data_as(_lib._PU32) if len(ix) else None,
                                   self.batch_size,
                                   _lib.PLAN_CASCADE if cascade else _lib.PLAN_FLAT,
                                   C.byref(opt), C.byref(self._h)))
        self.workspace_size = lib().dh_plan_workspace_size(self._h)

    @classmethod
    def from_tree(cls, backend: Backend, config: AttentionConfig, pool: Pool, tree, nodes,
                  cascade: bool = True) -> "DecodePlan":
        """dh_plan_create_tree: a plan over tree nodes, their page lists read
        from the tree's block tables by the library."""
        self = cls.__new__(cls)
        self.backend, self.pool, self.config = backend, pool, config
        ns = np.ascontiguousarray(nodes, dtype=np.uint64)
        self.batch_size = len(ns)
        self._c = config.to_c()
        self._h = C.c_void_p()
        self._destroy = lib().dh_plan_destroy
        opt = _lib.dh_plan_options()
        check(lib().dh_plan_create_tree(backend._h, C.byref(self._c), pool._h, tree._h,
                                        ns.ctypes.data_as(_lib._PU64), len(ns),
                                        _lib.PLAN_CASCADE if cascade else _lib.PLAN_FLAT,
                                        C.byref(opt), C.byref(self._h)))
        self.workspace_size = lib().dh_plan_workspace_size(self._h)
        return self

    def __del__(self):
        # Bound at construction: module globals may already be gone when an
        # object is collected at interpreter shutdown.
        destroy = getattr(self, "_destroy", None)
        if destroy is not None and getattr(self, "_h", None) and self._h.value:
            destroy(self._h)
            self._h = None

    def update(self, events, stream=None) -> bool:
        """dh_plan_update: apply [(sequence, op, page_id)] (op PLAN_APPEND or
        PLAN_REPLACE_LAST) in place on the stream; False when they do not fit
        and a new plan is needed (nothing changed then)."""
        ev = np.asarray(list(events), dtype=np.uint32).reshape(-1, 3)
        seqs, ops, ids = (np.ascontiguousarray(ev[:, i]) for i in range(3))
        patched = C.c_uint32()
        check(lib().dh_plan_update(self._h, len(ev), seqs.ctypes.data_as(_lib._PU32),
                                   ops.ctypes.data_as(_lib._PU32), ids.ctypes.data_as(_lib._PU32),
                                   C.c_void_p(_stream_ptr(stream)), C.byref(patched)))
        return bool(patched.value)

    def stats(self) -> dict:
        s = _lib.dh_plan_stats()
        check(lib().dh_plan_get_stats(self._h, C.byref(s)))
        return {k: getattr(s, k) for k, _ in s._fields_}

    def workspace(self):
        torch = _torch()
        return torch.empty(max(256, self.workspace_size), dtype=torch.uint8,
                           device=f"cuda:{self.backend.device}")


def plan_inspect(config: AttentionConfig, num_pool_pages: int, indptr, indices, cascade: bool = True,
                 shared_chunk_pages: int = 0, private_chunk_pages: int = 0,
                 target_items: int = 0, direct: bool = True) -> dict:
    """Host-only planning (dh_plan_inspect): the plan's stats, items, page list
    and (sequence, slot) pairs, without a device."""
    ip = np.ascontiguousarray(indptr, dtype=np.uint32)
    ix = np.ascontiguousarray(indices, dtype=np.uint32)
    batch = len(ip) - 1
    opt = _lib.dh_plan_options()
    opt.shared_chunk_pages = shared_chunk_pages
    opt.private_chunk_pages = private_chunk_pages
    opt.target_items = target_items
    opt.direct = _lib.DIRECT_AUTO if direct else _lib.DIRECT_OFF
    c = config.to_c()
    flags = _lib.PLAN_CASCADE if cascade else _lib.PLAN_FLAT
    ni, npg, nss = C.c_uint32(), C.c_uint32(), C.c_uint32()
    st = _lib.dh_plan_stats()
    args = (C.byref(c), num_pool_pages, ip.ctypes.data_as(_lib._PU32),
            ix.ctypes.data_as(_lib._PU32) if len(ix) else None, batch, flags, C.byref(opt))
    check(lib().dh_plan_inspect(*args, C.byref(st), None, C.byref(ni), None, C.byref(npg), None,
                                C.byref(nss)))
    items = (_lib.dh_plan_item * max(1, ni.value))()
    pages = np.zeros(max(1, npg.value), dtype=np.uint32)
    ss = np.zeros(2 * max(1, nss.value), dtype=np.uint32)
    check(lib().dh_plan_inspect(*args, C.byref(st), items, C.byref(ni), pages.ctypes.data_as(_lib._PU32),
                                C.byref(npg), ss.ctypes.data_as(_lib._PU32), C.byref(nss)))
    fields = [f for f, _ in _lib.dh_plan_item._fields_]
    return {"stats": {k: getattr(st, k) for k, _ in st._fields_},
            "items": [{f: getattr(items[i], f) for f in fields} for i in range(ni.value)],
            "pages": pages[:npg.value], "seqslots": ss[:2 * nss.value].reshape(-1, 2)}


class PrefillPlan(DecodePlan):
    """dh_plan_create_prefill: attention of each sequence's last q_len tokens
    over its kv_len paged tokens, causal (bottom-right aligned) or full; run
    with decode_batch on q / out of [sum(q_len), num_heads, head_dim]."""

    def __init__(self, backend: Backend, config: AttentionConfig, pool: Pool, indptr, indices, kv_len, q_len,
                 causal: bool = True, chunk_pages: int = 0):
        self.backend = backend
        self.pool = pool
        self.config = config
        ip = np.ascontiguousarray(indptr, dtype=np.uint32)
        ix = np.ascontiguousarray(indices, dtype=np.uint32)
        kv = np.ascontiguousarray(kv_len, dtype=np.uint32)
        ql = np.ascontiguousarray(q_len, dtype=np.uint32)
        self.batch_size = len(ip) - 1
        self.num_queries = int(ql.sum())
        self._c = config.to_c()
        self._h = C.c_void_p()
        self._destroy = lib().dh_plan_destroy
        check(lib().dh_plan_create_prefill(backend._h, C.byref(self._c), pool._h, ip.ctypes.data_as(_lib._PU32),
                                           ix.ctypes.data_as(_lib._PU32) if len(ix) else None,
                                           kv.ctypes.data_as(_lib._PU32), ql.ctypes.data_as(_lib._PU32),
                                           self.batch_size, int(causal), chunk_pages, C.byref(self._h)))
        self.workspace_size = lib().dh_plan_workspace_size(self._h)


def decode_batch(plan: DecodePlan, q, out, workspace, last_page_len=None, stream=None,
                 stages: int = 3) -> None:
    """One decode step through dh_decode_stages (stages=3 is dh_decode_batch).
    q, out: device tensors [B][Hq][D]; last_page_len: device int32 [B] or None."""
    lpl = None if last_page_len is None else C.c_void_p(last_page_len.data_ptr())
    check(lib().dh_decode_stages(plan.backend._h, plan.pool._h, plan._h, C.c_void_p(q.data_ptr()),
                                 lpl, C.c_void_p(out.data_ptr()), C.c_void_p(workspace.data_ptr()),
                                 workspace.numel() * workspace.element_size(), stages,
                                 C.c_void_p(_stream_ptr(stream))))


def decode_batch_host_lens(plan: DecodePlan, q, out, workspace, last_page_len=None, stream=None) -> None:
    """dh_decode_batch_host_lens: dh_decode_batch with the last-page lengths
    a host int32 array (numpy, or None: all pages full), carried to the
    kernels in their arguments; at most HOST_LENS_MAX_BATCH sequences."""
    lpl = None
    if last_page_len is not None:
        last_page_len = np.ascontiguousarray(last_page_len, dtype=np.int32)
        lpl = C.c_void_p(last_page_len.ctypes.data)
    check(lib().dh_decode_batch_host_lens(plan.backend._h, plan.pool._h, plan._h, C.c_void_p(q.data_ptr()), lpl,
                                          C.c_void_p(out.data_ptr()), C.c_void_p(workspace.data_ptr()),
                                          workspace.numel() * workspace.element_size(),
                                          C.c_void_p(_stream_ptr(stream))))


def csr_workspace_size(config: AttentionConfig, batch_size: int, max_total_pages: int) -> int:
    """dh_csr_workspace_size: workspace bytes of decode_csr."""
    return int(lib().dh_csr_workspace_size(C.byref(config.to_c()), batch_size, max_total_pages))


def decode_csr(backend: "Backend", pool: "Pool", config: AttentionConfig, q, indices, indptr, last_page_len,
               out, workspace, status=None, stream=None) -> None:
    """dh_decode_csr: one decode step from device int32 CSR page tables
    (BatchDecodeKernel::run, batch_decode.rs:86-95).  q / out [B][Hq][D];
    indices, indptr, last_page_len (or None), status (or None): device int32
    tensors; workspace: device uint8 of >= csr_workspace_size bytes."""
    batch = int(indptr.numel()) - 1
    ptr = lambda t: None if t is None else C.c_void_p(t.data_ptr())  # noqa: E731
    check(lib().dh_decode_csr(backend._h, pool._h, C.byref(config.to_c()), max(batch, 0), ptr(q), ptr(indices),
                              ptr(indptr), ptr(last_page_len), ptr(out), ptr(workspace),
                              workspace.numel() * workspace.element_size(), ptr(status),
                              C.c_void_p(_stream_ptr(stream))))


class TreeDecoder:
    """Decode steps over the leaves of a TreeState (tree/state.rs) with one
    cascade plan kept current from the tree's own events.

    append_token(i, token) runs TreeState::append_token on leaf i
    (tree/state.rs:87-113) and records what it did to the leaf's page list:
    a block allocated on a block boundary (PLAN_APPEND), or the copy-on-write
    of a shared partial last block, whose page data it copies
    (dh_pool_copy_page) before recording PLAN_REPLACE_LAST.  It returns
    (page, offset) where the new token's K / V go; writing them is the
    caller's (append_kv).  fork(i) adds a leaf (TreeState::fork, :49-84).
    decode(q) applies the recorded events to the plan in place
    (dh_plan_update) and builds a new plan from the tree's block tables only
    when they do not fit or the set of leaves changed.  Leaves are the plan's
    sequences, in order; q / out are device tensors [leaves][Hq][D]."""

    def __init__(self, backend: Backend, pool: Pool, tree, config: AttentionConfig, leaves):
        if tree.tokens_per_block != _lib.PAGE_SIZE:
            raise DhError(_lib.DH_EUNSUPPORTED,
                          f"TreeDecoder needs a tree of {_lib.PAGE_SIZE}-token blocks "
                          f"(this one has {tree.tokens_per_block})")
        self.backend = backend
        self.pool = pool
        self.tree = tree
        self.config = config
        self.leaves = [int(n) for n in leaves]
        # Each leaf's last page (where its next token goes unless the tree
        # allocates or copies a block), so an append reads no block table.
        self._last = [self._table_last(n) for n in self.leaves]
        self._plan: Optional[DecodePlan] = None
        self._ws = None
        self._events: list[tuple[int, int, int]] = []
        self._lpl = None    # last decode's device last_page_len, alive until the next decode
        self.plans_built = 0
        self.plans_patched = 0

    def _table_last(self, node: int) -> int:
        table = self.tree.get_block_table(node) or []
        return int(table[-1]) if table else _lib.INVALID_PAGE

    def fork(self, i: int) -> int:
        """Forks leaf i into a new leaf (appended last); returns its index."""
        self.leaves.append(int(self.tree.fork(self.leaves[i]).node_id))
        self._last.append(self._last[i])          # the child shares the parent's blocks
        self._plan = None
        return len(self.leaves) - 1

    def append_token(self, i: int, token: int, stream=None) -> tuple[int, int]:
        node = self.leaves[i]
        n = self.tree.get_node(node).num_tokens
        cow = self.tree.append_token(node, token)
        if n % _lib.PAGE_SIZE == 0:               # a new block at the end
            self._last[i] = self._table_last(node)
            self._events.append((i, _lib.PLAN_APPEND, self._last[i]))
        elif cow is not None:                     # the shared last block copied
            self.pool.copy_page(int(cow[0]), int(cow[1]), stream)
            self._last[i] = int(cow[1])
            self._events.append((i, _lib.PLAN_REPLACE_LAST, self._last[i]))
        return self._last[i], n % _lib.PAGE_SIZE

    def tables(self) -> list[list[int]]:
        return [[int(b) for b in self.tree.get_block_table(n)] for n in self.leaves]

    def last_page_len(self) -> np.ndarray:
        ns = np.ascontiguousarray(self.leaves, dtype=np.uint64)
        out = np.zeros(len(ns), np.int32)
        check(lib().dh_tree_last_page_len(self.tree._h, ns.ctypes.data_as(_lib._PU64), len(ns),
                                          out.ctypes.data_as(C.POINTER(C.c_int32))))
        return out

    def decode(self, q, out=None, stream=None):
        torch = _torch()
        if self._plan is not None and self._events:
            if self._plan.update(self._events, stream):
                self.plans_patched += 1
            else:
                self._plan = None
        self._events = []
        if self._plan is None:
            self._plan = DecodePlan.from_tree(self.backend, self.config, self.pool, self.tree, self.leaves)
            self._ws = self._plan.workspace()
            self.plans_built += 1
        dev = f"cuda:{self.backend.device}"
        if out is None:
            out = torch.empty_like(q)
        # The lengths are copied on the decode's stream and kept on self until
        # the next decode: the caching allocator cannot hand their memory to
        # another tensor while the kernels may still read it.
        with torch.cuda.stream(_as_torch_stream(stream)):
            self._lpl = torch.from_numpy(self.last_page_len()).to(dev)   # 0 reads as a full page
        decode_batch(self._plan, q, out, self._ws, self._lpl, stream)
        return out


def _list_events(old: np.ndarray, new: np.ndarray):
    """dh_plan_update events turning page list old into new: [] when equal;
    appends when new extends old; a replaced last page (copy-on-write)
    followed by appends.  None for anything else (a new plan)."""
    n = min(len(old), len(new))
    same = int(np.argmin(old[:n] == new[:n])) if n and not (old[:n] == new[:n]).all() else n
    if same == len(old) and len(new) >= len(old):
        return [(_lib.PLAN_APPEND, int(p)) for p in new[same:]]
    if len(old) and same == len(old) - 1 and len(new) >= len(old):
        return [(_lib.PLAN_REPLACE_LAST, int(new[same]))] + [(_lib.PLAN_APPEND, int(p)) for p in new[same + 1:]]
    return None


def _batched(queries, shape, dev):
    """(the queries as one [B][H][D] tensor, whether it is a view): a view
    when they already are consecutive rows of one buffer, else a stacked
    copy."""
    torch = _torch()
    q0 = queries[0]
    B, H, D = shape
    step = H * D
    if q0.is_cuda and q0.is_contiguous():
        base = q0.data_ptr()
        es = q0.element_size()
        if all(x.is_contiguous() and x.dtype == q0.dtype and x.data_ptr() == base + i * step * es
               and x.numel() == step for i, x in enumerate(queries)):
            st = q0.untyped_storage()
            off = q0.storage_offset()
            if off + B * step <= st.nbytes() // es:
                return torch.empty(0, dtype=q0.dtype, device=q0.device).set_(st, off, (B, H, D)), True
    return torch.stack([x.reshape(H, D) for x in queries]).to(dev).contiguous(), False


class _PageLens(dict):
    """block id -> tokens stored, kept in step with `array` (int32 over the
    pool) and `epoch` (moves when a block starts or stops holding tokens)."""

    def __init__(self, num_pages: int):
        super().__init__()
        self.array = np.zeros(num_pages, dtype=np.int32)
        self.epoch = 0

    def _mirror(self, block, n) -> None:
        b = int(block)
        old = int(self.array[b]) if 0 <= b < len(self.array) else int(dict.get(self, b, 0))
        if 0 <= b < len(self.array):
            self.array[b] = n
        if (old > 0) != (n > 0):
            self.epoch += 1

    def __setitem__(self, block, n) -> None:
        self._mirror(block, int(n))
        super().__setitem__(block, n)

    def __delitem__(self, block) -> None:
        self._mirror(block, 0)
        super().__delitem__(block)

    def pop(self, block, *default):
        if block in self:
            self._mirror(block, 0)
        return super().pop(block, *default)

    def clear(self) -> None:
        super().clear()
        self.array[:] = 0
        self.epoch += 1

    def update(self, *a, **kw) -> None:
        for k, v in dict(*a, **kw).items():
            self[k] = v

    def setdefault(self, block, n=None):
        if block not in self:
            self[block] = n
        return self[block]


class _PlanCache:
    """HipBackend's decode plan and what goes with it across calls: the key
    it was built for, each sequence's page list and last page, the
    workspace, and a ring of pinned host buffers for last_page_len (a
    buffer is refilled only after the copy that read it has run)."""

    RING = 4

    def __init__(self):
        self.key = None
        self.mut = -1
        self.tables = []
        self.cfg = None
        self.plan = None
        self.ws = None
        self.kept = []
        self.last_ids = np.zeros(0, dtype=np.int64)
        self.last_empty = np.zeros(0, dtype=bool)
        self._queries = None     # the last call's query list and its batched tensor
        self._qbatch = None
        self._retired = []   # (plan, event): freed once the work that read it has run
        self._host = []
        self._dev = []
        self._done = []
        self._i = 0

    def replace(self, plan) -> None:
        """Makes plan current; the previous one lives until the work already
        queued on the current stream (which may read it) has run."""
        torch = _torch()
        self._retired = [(p, e) for p, e in self._retired if not e.query()]
        if self.plan is not None:
            ev = torch.cuda.Event()
            ev.record()
            self._retired.append((self.plan, ev))
        self.plan = plan

    def new_batch(self, batch: int, device: int) -> None:
        torch = _torch()
        if self._host and self._host[0].numel() == batch:
            return
        self._host = [torch.empty(batch, dtype=torch.int32, pin_memory=True) for _ in range(self.RING)]
        self._dev = [torch.empty(batch, dtype=torch.int32, device=f"cuda:{device}") for _ in range(self.RING)]
        self._done = [torch.cuda.Event() for _ in range(self.RING)]
        self._used = [False] * self.RING

    def query_batch(self, queries, shape, dev):
        """_batched, skipped when the call passes the very tensors of the
        previous call and those were a view of one buffer (a serving loop's
        persistent query rows: the view sees their new contents)."""
        prev = self._queries
        if prev is not None and len(prev) == len(queries) and all(a is b for a, b in zip(prev, queries)):
            return self._qbatch
        q, view = _batched(queries, shape, dev)
        self._queries, self._qbatch = (list(queries), q) if view else (None, None)
        return q

    def last_page_lens(self, values):
        i = self._i
        self._i = (i + 1) % self.RING
        if self._used[i]:
            self._done[i].synchronize()
        self._host[i].numpy()[:] = values
        self._dev[i].copy_(self._host[i], non_blocking=True)
        self._done[i].record()
        self._used[i] = True
        return self._dev[i]


class HipBackend:
    """AttentionBackend (backend.rs:61-97) on the HIP decode path.

    Like ReferenceBackend it owns a KV store keyed by physical block id: here a
    device page pool.  append_kv writes tokens into the page of
    block_table[position / 16] at offset position % 16 (a whole 16-token block
    at position 16*b is exactly ReferenceBackend::append_kv's store); decode
    gathers the stored pages of each table, skipping INVALID and never-written
    blocks as ReferenceBackend skips blocks it has no KV for."""

    def __init__(self, device: int = 0, num_pages: int = 4096, num_kv_heads: int = 8,
                 head_dim: int = 128, kv_format: int = _lib.KV_BF16, cascade: bool = True):
        self.backend = Backend(device)
        self.pool = Pool(self.backend, num_pages, num_kv_heads, head_dim, kv_format)
        self.cascade = cascade
        # Tokens stored per block (a dict, mirrored into an array over the
        # pool with an epoch that moves whenever a block starts or stops
        # holding tokens: what decode's page lists depend on, beyond the
        # tables themselves).
        self.page_len = _PageLens(num_pages)
        # FP8 pools: the f32 tokens of each page still being filled, so an
        # append re-quantises the page from all its tokens (a block scale
        # covers the whole page); dropped once the page holds 16 tokens.
        self._shadow: dict = {}
        # One plan cache per stream: a stream's calls run in order, so its
        # cached plan may be patched and its workspace reused by the next
        # call on it, while calls on another stream get their own plan and
        # workspace.  The lock serialises the host side of the calls (plan
        # lookup, patching, launch), as the reference's backends guard
        # their state for &self access from several threads.
        self._plans: dict = {}
        self._lock = threading.RLock()
        self.plans_built = 0
        self.plans_patched = 0
        self.plans_reused = 0

    def _set_len(self, block: int, n: int) -> None:
        if n > 0:
            self.page_len[block] = n
        else:
            self.page_len.pop(block, None)

    @classmethod
    def new(cls, **kw) -> "HipBackend":
        return cls(**kw)

    def _append_quantised(self, page: int, off: int, key, value) -> int:
        """Writes tokens off.. of an FP8 / MXFP8 page: the page's f32 tokens
        so far plus these, quantised on the device (Pool.write_pages_device)."""
        torch = _torch()
        dev = f"cuda:{self.backend.device}"
        k, v = key.detach(), value.detach()
        if k.dim() == 4:
            k, v = k[0], v[0]
        hkv, d = self.pool.num_kv_heads, self.pool.head_dim
        n = k.shape[1]
        if tuple(k.shape) != (hkv, n, d) or tuple(v.shape) != (hkv, n, d) or off + n > _lib.PAGE_SIZE:
            raise DhError(_lib.DH_EINVAL, f"key shape {tuple(key.shape)} at offset {off} does not fit the page")
        sh = self._shadow.get(page)
        if off == 0 or sh is None:
            if off != 0 and self.page_len.get(page, 0) > 0:
                raise DhError(_lib.DH_EUNSUPPORTED, f"FP8 page {page} is complete; rewrite it from offset 0")
            sh = torch.zeros((1, 2, hkv, _lib.PAGE_SIZE, d), dtype=torch.float32, device=dev)
        sh[0, 0, :, off:off + n] = k.to(dev, torch.float32)
        sh[0, 1, :, off:off + n] = v.to(dev, torch.float32)
        # On the current stream, after the shadow's updates and before any
        # later use of it or of the id tensor's memory: no host wait.
        self.pool.write_pages_device(torch.tensor([page], dtype=torch.int32, device=dev), sh)
        if off + n == _lib.PAGE_SIZE:
            self._shadow.pop(page, None)
        else:
            self._shadow[page] = sh
        return n

    def _kv_np(self, t) -> np.ndarray:
        torch = _torch()
        want = {_lib.KV_F16: torch.float16, _lib.KV_BF16: torch.bfloat16,
                _lib.KV_F32: torch.float32}.get(self.pool.kv_format)
        if want is None:
            raise DhError(_lib.DH_EUNSUPPORTED, "append_kv of FP8 pages needs pre-quantised pages "
                          "(use Pool.write_tokens)")
        t = t.detach().to("cpu").to(want).contiguous()
        if t.dim() == 4:
            t = t[0]
        return t.view(torch.int16 if want != torch.float32 else torch.int32).numpy()

    def append_kv(self, key, value, block_table: BlockTable, position: int) -> None:
        """key/value: [1, num_kv_heads, n, head_dim]; n + position % 16 <= 16."""
        with self._lock:
            self._append_kv(key, value, block_table, position)

    def _append_kv(self, key, value, block_table: BlockTable, position: int) -> None:
        block = block_table.get(position // _lib.PAGE_SIZE)
        if block is None or not block.is_valid():
            return                                   # backend.rs:296-298: no block, no store
        off = position % _lib.PAGE_SIZE
        stored = self.page_len.get(int(block), 0)
        if off > stored:
            # Tokens [stored, off) of the page were never written (a fresh
            # page, or one forgotten by clear_cache): attending to them would
            # read zeros or stale K/V.  The reference's store keeps only the
            # given tokens (backend.rs:285-301); writes here go to their
            # offset, so the page must be filled from the front.
            raise DhError(_lib.DH_EUNSUPPORTED,
                          f"append_kv at position {position}: block {int(block)} holds {stored} tokens, "
                          f"so offset {off} would leave tokens {stored}..{off - 1} unwritten")
        if self.pool.kv_format in (_lib.KV_FP8_E4M3, _lib.KV_MXFP8):
            n = self._append_quantised(int(block), off, key, value)
            self._set_len(int(block), max(self.page_len.get(int(block), 0), off + n))
            return
        k = self._kv_np(key)
        v = self._kv_np(value)
        if k.shape[0] != self.pool.num_kv_heads or k.shape[2] != self.pool.head_dim:
            raise DhError(_lib.DH_EINVAL, f"key shape {tuple(key.shape)} does not match the pool")
        self.pool.write_tokens(int(block), off, k, v)
        self._set_len(int(block), max(self.page_len.get(int(block), 0), off + k.shape[1]))

    def store_kv(self, block_id: int, key, value) -> None:
        """ReferenceBackend::store_kv (backend.rs:140-143): the block's entry
        becomes key / value ([1, num_kv_heads, n, head_dim], n <= 16), from
        token 0 (overwrite, as the reference's map insert)."""
        with self._lock:
            self._set_len(int(block_id), 0)
            self._shadow.pop(int(block_id), None)
            self._append_kv(key, value, BlockTable.from_blocks([int(block_id)]), 0)

    def get_kv(self, block_id: int):
        """ReferenceBackend::get_kv (backend.rs:135-138): the stored K and V of
        a block as host tensors [1, num_kv_heads, n, head_dim] of the pool's
        element type, or None when nothing is stored.  FP8 / MXFP8 pages hold
        codes and scales (Pool.read_page), not elements: DH_EUNSUPPORTED."""
        torch = _torch()
        n = self.page_len.get(int(block_id), 0)
        if n == 0:
            return None
        fmt = self.pool.kv_format
        if fmt in (_lib.KV_FP8_E4M3, _lib.KV_MXFP8):
            raise DhError(_lib.DH_EUNSUPPORTED, "FP8 / MXFP8 pages hold codes and scales: use Pool.read_page")
        dt = {_lib.KV_F32: torch.float32, _lib.KV_BF16: torch.bfloat16, _lib.KV_F16: torch.float16}[fmt]
        raw, _ = self.pool.read_page(int(block_id))
        hkv, d = self.pool.num_kv_heads, self.pool.head_dim
        t = torch.from_numpy(raw.copy()).view(dt).reshape(2, hkv, _lib.PAGE_SIZE, d)[:, :, :n]
        return t[0:1].contiguous(), t[1:2].contiguous()

    def clear_cache(self) -> None:
        """ReferenceBackend::clear_cache (backend.rs:130-133): every stored
        block is forgotten (decode then skips them, as blocks with no KV)."""
        with self._lock:
            self.page_len.clear()
            self._shadow.clear()

    def _kept(self, t: BlockTable) -> np.ndarray:
        """The table's pages decode reads: valid blocks holding tokens, in
        order; every one but the last must be full."""
        ids = t.block_ids()
        lens = self.page_len.array
        inpool = ids < len(lens)
        kept = ids[inpool & (lens[np.where(inpool, ids, 0)] > 0)]
        if len(kept) > 1:
            short = lens[kept[:-1]] != _lib.PAGE_SIZE
            if short.any():
                b = int(kept[:-1][short][0])
                raise DhError(_lib.DH_EUNSUPPORTED,
                              f"block {b} holds {self.page_len[b]} tokens but is not the last "
                              "stored block of its table")
        return kept

    def _csr(self, tables: Sequence[BlockTable]):
        kept = [self._kept(t) for t in tables]
        indptr = np.concatenate([[0], np.cumsum([len(k) for k in kept])]).astype(np.uint32)
        indices = np.concatenate(kept).astype(np.uint32) if kept else np.zeros(0, np.uint32)
        lpl = np.array([self.page_len[int(k[-1])] if len(k) else _lib.PAGE_SIZE for k in kept], dtype=np.int32)
        return indptr, indices, lpl

    def _plan_for(self, c: "_PlanCache", tables: Sequence[BlockTable], cfg: AttentionConfig, cfg_key):
        """The decode plan of these tables in the stream's cache c: the
        cached one when neither the tables (uid, version) nor the set of
        stored blocks changed; patched in place (dh_plan_update) when each
        page list only gained pages at its end or had its last page
        replaced; else a new plan."""
        from .cache import block_table_mutations
        mut = block_table_mutations()
        if (c.plan is not None and c.mut == mut and c.key[0] == cfg_key and c.key[3] == self.page_len.epoch
                and len(c.tables) == len(tables) and all(a is b for a, b in zip(c.tables, tables))):
            self.plans_reused += 1     # no table changed anywhere since the plan's key was taken
            return c
        key = (cfg_key, tuple(t.uid for t in tables), tuple(t.version for t in tables), self.page_len.epoch)
        if c.plan is not None and c.key == key:
            c.mut, c.tables = mut, list(tables)
            self.plans_reused += 1
            return c
        kept = [self._kept(t) for t in tables]
        events = None
        if c.plan is not None and c.key[0] == cfg_key and c.key[1] == key[1]:
            events = []
            for i, (old, new) in enumerate(zip(c.kept, kept)):
                ev = _list_events(old, new)
                if ev is None:
                    events = None
                    break
                events.extend((i, op, pid) for op, pid in ev)
        if events is not None and (not events or c.plan.update(events)):
            self.plans_patched += bool(events)
            self.plans_reused += not events
        else:
            indptr = np.concatenate([[0], np.cumsum([len(k) for k in kept])]).astype(np.uint32)
            indices = np.concatenate(kept).astype(np.uint32) if kept else np.zeros(0, np.uint32)
            c.replace(DecodePlan(self.backend, cfg, self.pool, indptr, indices, cascade=self.cascade))
            if c.ws is None or c.ws.numel() < c.plan.workspace_size:
                c.ws = c.plan.workspace()
            c.new_batch(len(tables), self.backend.device)
            self.plans_built += 1
        c.key = key
        c.mut, c.tables = mut, list(tables)
        c.kept = kept
        c.last_ids = np.array([int(k[-1]) if len(k) else 0 for k in kept], dtype=np.int64)
        c.last_empty = np.array([len(k) == 0 for k in kept], dtype=bool)
        return c

    def decode_batch(self, queries, block_tables: Sequence[BlockTable], config: AttentionConfig):
        """queries: list of [1, num_heads, 1, head_dim] tensors; returns the
        outputs as one tensor [B, 1, num_heads, 1, head_dim] of the queries'
        dtype, whose row i is query i's output (indexed and iterated like the
        reference's Vec<Tensor>, backend.rs:267-283).  The plan is cached
        across calls (see _plan_for); the sequences' last-page lengths go up
        through pinned host buffers.  Results are ordered on the current
        stream (no host synchronisation)."""
        torch = _torch()
        if len(queries) != len(block_tables):
            raise DhError(_lib.DH_EINVAL, "queries and block_tables differ in length")
        if not queries:
            return []
        dev = f"cuda:{self.backend.device}"
        qdt = queries[0].dtype
        cfg_key = (config.num_heads, config.num_kv_heads, config.head_dim, config.scale, config.gqa_mapping, qdt)
        stream = _stream_ptr(None)
        with self._lock:
            c = self._plans.get(stream)
            if c is None:
                c = self._plans[stream] = _PlanCache()
            cfg = c.cfg if c.key is not None and c.key[0] == cfg_key else None
            if cfg is None:
                cfg = AttentionConfig(config.num_heads, config.num_kv_heads, config.head_dim)
                cfg.scale = config.scale
                cfg.sliding_window = config.sliding_window
                cfg.gqa_mapping = config.gqa_mapping
                cfg.q_dtype = dtype_code(qdt)
                cfg.kv_format = self.pool.kv_format
            c = self._plan_for(c, block_tables, cfg, cfg_key)
            c.cfg = cfg
            B, H, D = len(queries), config.num_heads, config.head_dim
            q = c.query_batch(queries, (B, H, D), dev)
            lens = self.page_len.array[c.last_ids]
            lens[c.last_empty] = _lib.PAGE_SIZE
            out = torch.empty((B, H, D), dtype=qdt, device=dev)
            if B <= _lib.HOST_LENS_MAX_BATCH:    # lengths in the kernel arguments: no upload, no event
                decode_batch_host_lens(c.plan, q, out, c.ws, lens, stream=stream)
            else:
                decode_batch(c.plan, q, out, c.ws, c.last_page_lens(lens), stream=stream)
        return out.view(B, 1, H, 1, D)

    def decode(self, query, block_table: BlockTable, config: AttentionConfig):
        """backend.rs:206-265."""
        return self.decode_batch([query], [block_table], config)[0]

    def prefill(self, query, key, value, block_table: BlockTable, config: AttentionConfig):
        """ReferenceBackend::prefill (backend.rs:163-204): causal attention of
        query [B, num_heads, S, head_dim] over key / value [B, num_kv_heads,
        S, head_dim] (GQA per config), output like query.  As there, the block
        table is not read: K / V are staged in a temporary pool of the query's
        dtype and run through a prefill plan (q_len = kv_len = S).  float32
        queries (the prefill kernel is 16-bit) run as a decode over one
        virtual sequence per query, its page list cut after the query's own
        token: the cascade plan reads the nested shared prefixes once."""
        torch = _torch()
        dev = f"cuda:{self.backend.device}"
        if query.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise DhError(_lib.DH_EUNSUPPORTED, "prefill takes float32, bf16 or f16 queries")
        bsz, hq, S, d = query.shape
        hkv = key.shape[1]
        if tuple(key.shape) != (bsz, hkv, S, d) or tuple(value.shape) != tuple(key.shape):
            raise DhError(_lib.DH_EINVAL, f"key / value shape {tuple(key.shape)} does not match the query")
        if S == 0 or bsz == 0:
            return torch.zeros_like(query)
        npg = (S + _lib.PAGE_SIZE - 1) // _lib.PAGE_SIZE
        fmt = {torch.bfloat16: _lib.KV_BF16, torch.float16: _lib.KV_F16, torch.float32: _lib.KV_F32}[query.dtype]
        pool = Pool(self.backend, bsz * npg, hkv, d, fmt)
        pad = npg * _lib.PAGE_SIZE - S
        kv = torch.stack([key, value], dim=1).to(dev, query.dtype)            # [B, 2, Hkv, S, D]
        kv = torch.nn.functional.pad(kv, (0, 0, 0, pad))                       # [B, 2, Hkv, npg*16, D]
        src = kv.reshape(bsz, 2, hkv, npg, _lib.PAGE_SIZE, d).permute(0, 3, 1, 2, 4, 5).contiguous()
        src = src.reshape(bsz * npg, 2, hkv, _lib.PAGE_SIZE, d)
        pool.write_pages_device(torch.arange(bsz * npg, dtype=torch.int32, device=dev), src)
        cfg = AttentionConfig(config.num_heads, config.num_kv_heads, config.head_dim)
        cfg.scale = config.scale
        cfg.gqa_mapping = config.gqa_mapping
        cfg.q_dtype = dtype_code(query.dtype)
        cfg.kv_format = fmt
        q = query.to(dev).permute(0, 2, 1, 3).reshape(bsz * S, hq, d).contiguous()
        out = torch.empty_like(q)
        if fmt == _lib.KV_F32:
            # query i of sequence b sees tokens 0 .. i: pages 0 .. i // 16 of
            # b's, the last holding i % 16 + 1 of them
            i = np.arange(S)
            per = i // _lib.PAGE_SIZE + 1
            indptr = np.concatenate([[0], np.cumsum(np.tile(per, bsz))]).astype(np.uint32)
            indices = np.concatenate([b * npg + np.arange(n) for b in range(bsz) for n in per]).astype(np.uint32)
            lpl = torch.from_numpy(np.tile(i % _lib.PAGE_SIZE + 1, bsz).astype(np.int32)).to(dev)
            plan = DecodePlan(self.backend, cfg, pool, indptr, indices, cascade=True)
            decode_batch(plan, q, out, plan.workspace(), lpl)
            torch.cuda.synchronize(dev)
            return out.reshape(bsz, S, hq, d).permute(0, 2, 1, 3).contiguous()
        indptr = np.arange(bsz + 1, dtype=np.uint32) * npg
        indices = np.arange(bsz * npg, dtype=np.uint32)
        lens = np.full(bsz, S, dtype=np.uint32)
        plan = PrefillPlan(self.backend, cfg, pool, indptr, indices, lens, lens, causal=True)
        decode_batch(plan, q, out, plan.workspace())
        torch.cuda.synchronize(dev)
        return out.reshape(bsz, S, hq, d).permute(0, 2, 1, 3).contiguous()


__all__ = ["AttentionConfig", "Backend", "Pool", "DecodePlan", "PrefillPlan", "decode_batch", "HipBackend",
           "is_available", "dtype_code", "torch_dtype", "raw_to_tensor"]
