"""dh_decode_batch_static, the entry point that allocates nothing: its
partial states go to the library's static per-GPU scratch array instead of a
caller workspace.  Checked through the C ABI against dh_decode_batch (the
same kernels, so the outputs must be bit-identical) on two calls in a row,
the second with a smaller batch, and a plan whose workspace exceeds the
array is refused with DH_ENOMEM."""
import ctypes as C

import numpy as np
import pytest
import torch

from dendrite_amd import _lib, workloads
from dendrite_amd._lib import lib
from dendrite_amd.backend import AttentionConfig, Backend, DecodePlan, Pool, decode_batch, raw_to_tensor

pytestmark = pytest.mark.gpu


def _static(plan, q, out, lpl):
    return lib().dh_decode_batch_static(plan.backend._h, plan.pool._h, plan._h, C.c_void_p(q.data_ptr()),
                                        C.c_void_p(lpl.data_ptr()), C.c_void_p(out.data_ptr()),
                                        C.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_static_decode_matches_workspace_decode():
    be = Backend(0)
    big = workloads.c3(root_pages=96, levels=3, level_pages=3, pool_pages=4096)
    small = workloads.c3(root_pages=24, levels=2, level_pages=2, pool_pages=4096)
    pool = Pool(be, big.num_pool_pages, big.hkv, big.d, big.kv_format)
    for w in (big, small):
        ids = w.page_ids()
        data, scales = w.make_pages(ids)
        pool.write_pages(ids, data, scales)
    for w in (big, small):            # two calls in a row, the second smaller
        cfg = w.attention_config()
        plan = DecodePlan(be, cfg, pool, w.indptr, w.indices, cascade=True)
        assert 0 < plan.workspace_size <= _lib.STATIC_WORKSPACE_BYTES
        q = raw_to_tensor(w.make_q(), w.q_dtype)
        lpl = torch.from_numpy(np.ascontiguousarray(w.last_page_len)).cuda()
        want = torch.empty_like(q)
        decode_batch(plan, q, want, plan.workspace(), lpl)
        got = torch.full_like(q, float("nan"))
        assert _static(plan, q, got, lpl) == _lib.DH_OK, C.string_at(lib().dh_last_error())
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), w.batch


def test_static_decode_refuses_plans_beyond_the_array():
    be = Backend(0)
    hq, hkv, d, n = 64, 8, 256, 1100           # 1100 slots x 64 heads x (256 x 2 + 8) B > 32 MiB
    pool = Pool(be, n, hkv, d, _lib.KV_BF16)
    cfg = AttentionConfig(hq, hkv, d)
    plan = DecodePlan(be, cfg, pool, np.arange(n + 1, dtype=np.uint32), np.arange(n, dtype=np.uint32),
                      cascade=False)
    assert plan.workspace_size > _lib.STATIC_WORKSPACE_BYTES
    q = torch.zeros((n, hq, d), dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    lpl = torch.full((n,), 16, dtype=torch.int32, device="cuda")
    assert _static(plan, q, out, lpl) == _lib.DH_ENOMEM
    assert b"static scratch" in C.string_at(lib().dh_last_error())
