"""Shared helpers: run a workload through the C ABI on the GPU and through the
CPU oracle on identical inputs."""
from __future__ import annotations

import numpy as np

import oracle
from dendrite_amd import _lib
from dendrite_amd.backend import Backend, DecodePlan, Pool, decode_batch, raw_to_tensor

TOL = {_lib.DTYPE_F32: 1e-4, _lib.DTYPE_BF16: 2e-2, _lib.DTYPE_F16: 2e-2}


def q_tensor(q_raw: np.ndarray, q_dtype: int, device: str = "cuda:0"):
    return raw_to_tensor(q_raw, q_dtype, device)


class GpuRun:
    """Uploads a workload's pages and runs one decode step."""

    def __init__(self, w, backend: Backend, cascade: bool = True, ids=None, scale=None, **plan_kw):
        import torch
        self.w = w
        self.backend = backend
        self.pool = Pool(backend, w.num_pool_pages, w.hkv, w.d, w.kv_format)
        self.ids = w.page_ids() if ids is None else ids
        self.data, self.scales = w.make_pages(self.ids)
        self.pool.write_pages(self.ids, self.data, self.scales)
        self.cfg = w.attention_config()
        if scale is not None:
            self.cfg.scale = float(scale)
        self.plan = DecodePlan(backend, self.cfg, self.pool, w.indptr, w.indices, cascade=cascade,
                               **plan_kw)
        self.q_raw = w.make_q()
        self.q = q_tensor(self.q_raw, w.q_dtype)
        self.out = torch.empty_like(self.q)
        self.ws = self.plan.workspace()
        self.lpl = torch.from_numpy(np.ascontiguousarray(w.last_page_len, dtype=np.int32)).to("cuda:0")

    def run(self) -> np.ndarray:
        import torch
        decode_batch(self.plan, self.q, self.out, self.ws, self.lpl)
        torch.cuda.synchronize()
        return self.out.float().cpu().numpy()

    def pool_view(self) -> oracle.PoolView:
        return oracle.PoolView(self.ids, self.data, self.scales, self.w.num_pool_pages,
                               self.w.kv_format, self.w.hkv, self.w.d)

    def reference(self, seqs=None) -> np.ndarray:
        w = self.w
        return oracle.decode(self.pool_view(), self.q_raw, w.q_dtype, w.hq, self.cfg.scale,
                             w.gqa_mapping, w.indptr, w.indices, w.last_page_len, seqs=seqs)


def max_abs_err(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.max(np.abs(got.astype(np.float64) - ref))) if got.size else 0.0


def half_ulp(ref: np.ndarray, q_dtype: int) -> np.ndarray:
    """Half a unit in the last place of the output dtype at |ref|: the error a
    correctly rounded output of that dtype already carries.  bf16 keeps 8
    significant bits, f16 11, f32 24."""
    bits = {_lib.DTYPE_BF16: 8, _lib.DTYPE_F16: 11, _lib.DTYPE_F32: 24}[q_dtype]
    a = np.maximum(np.abs(ref), np.finfo(np.float64).tiny)
    return np.ldexp(1.0, (np.floor(np.log2(a)).astype(np.int64) - bits))


def excess_err(got: np.ndarray, ref: np.ndarray, q_dtype: int) -> float:
    """max(|got - ref| - half_ulp(ref)): the error beyond the output dtype's own
    rounding.  The stated tolerances (f32 1e-4, bf16/FP8 2e-2 max-abs) are
    applied to this quantity, because a bf16 output above 8 in magnitude cannot
    be within 2e-2 of the exact value (its half-ulp there is >= 2^-5)."""
    if not got.size:
        return 0.0
    return float(np.max(np.abs(got.astype(np.float64) - ref) - half_ulp(ref, q_dtype)))
