"""Quantise-on-write on the device (dh_pool_write_pages_device) against the
oracle's page write rule (oracle_write_pages, pinned in
tests/test_oracle_write.py): bit-exact page data and scale records for every
pool format, source dtype and head_dim, with blocks that hold every E4M3 code
value and every tie between adjacent codes, values beyond the E4M3 range, an
all-zero block and a partial page; ids outside the pool skipped; and
HipBackend.append_kv into FP8 / MXFP8 pools (each append re-quantises the
page from all its tokens), decoded against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from dendrite_amd import _lib
from dendrite_amd.backend import AttentionConfig, HipBackend, Pool
from dendrite_amd.cache import BlockTable

pytestmark = pytest.mark.gpu

FMTS = [_lib.KV_F32, _lib.KV_BF16, _lib.KV_F16, _lib.KV_FP8_E4M3, _lib.KV_MXFP8]
FMT_IDS = ["f32", "bf16", "f16", "fp8", "mxfp8"]
SRC = [torch.float32, torch.bfloat16, torch.float16]


def _code_block(d):
    """16 x d values: every non-negative E4M3 code value, every midpoint of
    adjacent codes (ties), and their negatives; amax 448, so an FP8 block
    scale of 1 maps them onto the codes themselves."""
    vals = [oracle.e4m3_to_float(c) for c in range(0x7F)]
    mids = [(a + b) / 2 for a, b in zip(vals[:-1], vals[1:])]
    v = np.array(vals + mids + [-x for x in vals] + [-x for x in mids], dtype=np.float32)
    blk = np.zeros(16 * d, np.float32)
    blk[: min(v.size, blk.size)] = v[: blk.size]
    return blk.reshape(16, d)


def _pages(n, hkv, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 2, hkv, 16, d)).astype(np.float32)
    x[0, 0, 0] = _code_block(d)
    x[1, 1, hkv - 1] = 0.0                              # all-zero block
    m = rng.random(x[2].shape) < 0.02                   # outliers beyond the E4M3 range
    x[2][m] = np.where(x[2][m] < 0, -600.0, 600.0)
    x[3, :, :, 10:] = 0.0                               # a page of 10 tokens
    x[4] *= np.float32(1e-3)                            # small values (E4M3 subnormals at scale 1)
    return x


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("fmt", FMTS, ids=FMT_IDS)
@pytest.mark.parametrize("src_dtype", SRC, ids=["src_f32", "src_bf16", "src_f16"])
def test_device_write_matches_the_oracle(backend, d, fmt, src_dtype):
    hkv = 2 if d == 256 else 3
    print(f"[case] d={d} fmt={fmt} src={src_dtype}", flush=True)
    x = _pages(5, hkv, d, seed=d + fmt)
    src = torch.from_numpy(x).to(src_dtype)
    ref_data, ref_scales = oracle.write_pages(fmt, hkv, d, src.float().numpy())
    pool = Pool(backend, 40, hkv, d, fmt)
    ids = [7, 3, 39, 0, 21]
    pool.write_pages_device(torch.tensor(ids, dtype=torch.int32, device="cuda:0"), src.to("cuda:0"))
    torch.cuda.synchronize()
    for i, pid in enumerate(ids):
        data, scales = pool.read_page(pid)
        assert np.array_equal(data, ref_data[i]), f"page {i}: data differs from the oracle"
        if ref_scales is not None:
            assert np.array_equal(scales, ref_scales[i]), f"page {i}: scales differ from the oracle"


@pytest.mark.parametrize("fmt", [_lib.KV_BF16, _lib.KV_FP8_E4M3, _lib.KV_MXFP8], ids=["bf16", "fp8", "mxfp8"])
def test_ids_outside_the_pool_are_skipped(backend, fmt):
    hkv, d, n_pool = 2, 128, 8
    pool = Pool(backend, n_pool, hkv, d, fmt)
    before = np.random.default_rng(1).integers(0, 256, (n_pool, pool.page_bytes), dtype=np.uint8)
    if fmt == _lib.KV_FP8_E4M3:
        sb = np.ones((n_pool, 2 * hkv), np.float32).view(np.uint8)
    elif fmt == _lib.KV_MXFP8:
        sb = np.full((n_pool, pool.scale_bytes), 127, np.uint8)
    else:
        sb = None
    pool.write_pages(list(range(n_pool)), before, sb)
    x = _pages(5, hkv, d, seed=9)
    ids = torch.tensor([2, n_pool, 0xFFFFFFFF, 5, 1000], dtype=torch.uint32, device="cuda:0")
    pool.write_pages_device(ids, torch.from_numpy(x).to("cuda:0"))
    torch.cuda.synchronize()
    ref_data, ref_scales = oracle.write_pages(fmt, hkv, d, x)
    for pid in range(n_pool):
        data, scales = pool.read_page(pid)
        if pid == 2 or pid == 5:
            i = 0 if pid == 2 else 3
            assert np.array_equal(data, ref_data[i])
            if ref_scales is not None:
                assert np.array_equal(scales, ref_scales[i])
        else:
            assert np.array_equal(data, before[pid]), f"page {pid} was written"


@pytest.mark.parametrize("fmt", [_lib.KV_FP8_E4M3, _lib.KV_MXFP8], ids=["fp8", "mxfp8"])
def test_append_kv_quantises_on_the_device(fmt):
    """Token-by-token appends into an FP8 / MXFP8 pool end with the pages the
    write rule gives for the whole sequence, and decode matches the oracle on
    them (2e-2 beyond bf16 output rounding)."""
    from tests._helpers import TOL, excess_err
    hkv, d, hq, T = 2, 128, 8, 40
    be = HipBackend(num_pages=16, num_kv_heads=hkv, head_dim=d, kv_format=fmt)
    g = torch.Generator().manual_seed(2)
    k = torch.randn(hkv, T, d, generator=g)
    v = torch.randn(hkv, T, d, generator=g)
    table = BlockTable.from_blocks([4, 9, 1])
    pos = 0
    for step in (16, 1, 3, 7, 5, 8):                     # a whole block, then smaller appends
        n = min(step, 16 - pos % 16, T - pos)
        be.append_kv(k[None, :, pos:pos + n], v[None, :, pos:pos + n], table, pos)
        pos += n
    while pos < T:
        n = min(16 - pos % 16, T - pos)
        be.append_kv(k[None, :, pos:pos + n], v[None, :, pos:pos + n], table, pos)
        pos += n
    # expected pages: the write rule over each block's tokens (zeros past the end)
    blocks = [4, 9, 1]
    x = np.zeros((3, 2, hkv, 16, d), np.float32)
    for b in range(3):
        t0, t1 = 16 * b, min(16 * b + 16, T)
        x[b, 0, :, : t1 - t0] = k[:, t0:t1].numpy()
        x[b, 1, :, : t1 - t0] = v[:, t0:t1].numpy()
    ref_data, ref_scales = oracle.write_pages(fmt, hkv, d, x)
    for b, pid in enumerate(blocks):
        data, scales = be.pool.read_page(pid)
        assert np.array_equal(data, ref_data[b]), f"block {b} data"
        assert np.array_equal(scales, ref_scales[b]), f"block {b} scales"
    cfg = AttentionConfig(hq, hkv, d)
    q = torch.randn(1, hq, 1, d, generator=g).to(torch.bfloat16)
    out = be.decode(q, table, cfg)
    pv = oracle.PoolView(np.array(blocks, np.uint32), ref_data, ref_scales, 16, fmt, hkv, d)
    ref = oracle.decode(pv, q.float().reshape(1, hq, d).numpy(), _lib.DTYPE_F32, hq, cfg.scale, cfg.gqa_mapping,
                        np.array([0, 3], np.uint32), np.array(blocks, np.uint32),
                        np.array([T - 32], np.int32))
    got = out.float().reshape(1, hq, d).cpu().numpy()
    assert excess_err(got, ref, _lib.DTYPE_BF16) <= TOL[_lib.DTYPE_BF16]
