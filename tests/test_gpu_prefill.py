"""Paged prefill (dh_plan_create_prefill + dh_decode_batch) against the CPU
oracle: query i of a sequence with kv_len tokens and q_len queries sees the
first kv_len - q_len + i + 1 tokens (causal, bottom-right aligned) or all of
them, which is the decode oracle (oracle_decode, pinned in test_oracle.py) on
one virtual sequence per query whose page list is cut at that length.
Covers head_dim 64 / 128 / 256, bf16 / f16 / FP8 / MXFP8 KV, both GQA
mappings, chunked prefill over a cached context (q_len < kv_len), KV chunks
of a few pages (so rows span several partial states and the diagonal lands
inside and across chunks), INVALID ids, and HipBackend.prefill (the
reference's dense causal prefill).  Tolerance: 2e-2 beyond output rounding
(bf16 / f16 and FP8 after dequantisation), as for decode.
"""
import numpy as np
import pytest
import torch

import oracle
from dendrite_amd import _lib, workloads
from dendrite_amd.backend import AttentionConfig, HipBackend, Pool, PrefillPlan, decode_batch, raw_to_tensor
from tests._helpers import TOL, excess_err

pytestmark = pytest.mark.gpu


def _virtual(indptr, indices, kv_len, q_len, causal):
    """Per-query page lists and last-page lengths for the decode oracle."""
    vip, vix, vlpl = [0], [], []
    for b in range(len(kv_len)):
        pages = [int(p) for p in indices[indptr[b]:indptr[b + 1]] if p != _lib.INVALID_PAGE]
        for i in range(q_len[b]):
            n = kv_len[b] - q_len[b] + i + 1 if causal else kv_len[b]
            np_ = (n + 15) // 16
            vix.extend(pages[:np_])
            vip.append(len(vix))
            vlpl.append(n - 16 * (np_ - 1))
    return np.array(vip, np.uint32), np.array(vix, np.uint32), np.array(vlpl, np.int32)


def _run(backend, hq, hkv, d, q_dtype, fmt, kv_len, q_len, causal=True, chunk_pages=0, gqa=_lib.GQA_TILED,
         invalid=False, seed=0):
    rng = np.random.default_rng(seed)
    B = len(kv_len)
    npg = [(n + 15) // 16 for n in kv_len]
    pool_pages = sum(npg) + 8
    perm = rng.permutation(pool_pages).astype(np.uint32)
    indptr, indices, o = [0], [], 0
    for b in range(B):
        pg = list(perm[o:o + npg[b]])
        o += npg[b]
        if invalid and pg:
            pg.insert(len(pg) // 2, _lib.INVALID_PAGE)
        indices.extend(pg)
        indptr.append(len(indices))
    indptr, indices = np.array(indptr, np.uint32), np.array(indices, np.uint32)
    w = workloads.custom([[0]], hq, hkv, d, q_dtype, fmt, pool_pages, seed=seed + 77)
    ids = np.unique(indices[indices != _lib.INVALID_PAGE]).astype(np.uint32)
    data, scales = w.make_pages(ids)
    pool = Pool(backend, pool_pages, hkv, d, fmt)
    pool.write_pages(ids, data, scales)
    cfg = w.attention_config()
    cfg.gqa_mapping = gqa
    plan = PrefillPlan(backend, cfg, pool, indptr, indices, kv_len, q_len, causal=causal, chunk_pages=chunk_pages)
    nq = int(np.sum(q_len))
    qf = rng.standard_normal((nq, hq, d)).astype(np.float32)
    q = torch.from_numpy(qf).to(torch.bfloat16 if q_dtype == _lib.DTYPE_BF16 else torch.float16).to("cuda:0")
    out = torch.empty_like(q)
    decode_batch(plan, q, out, plan.workspace())
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    vip, vix, vlpl = _virtual(indptr, indices, kv_len, q_len, causal)
    pv = oracle.PoolView(ids, data, scales, pool_pages, fmt, hkv, d)
    ref = oracle.decode(pv, q.float().cpu().numpy(), _lib.DTYPE_F32, hq, cfg.scale, gqa, vip, vix, vlpl)
    err = excess_err(got, ref, q_dtype)
    print(f"[case] prefill hq={hq} hkv={hkv} d={d} fmt={fmt} kv={list(kv_len)} q={list(q_len)} "
          f"causal={causal} chunk={chunk_pages}: err {err:.3e} items {plan.stats()['num_items']}", flush=True)
    assert np.all(np.isfinite(got))
    assert err <= TOL[q_dtype], f"error beyond output rounding {err}"
    return plan


@pytest.mark.parametrize("shape", [(32, 8, 128), (16, 4, 64), (8, 2, 256), (32, 4, 64)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("fmt", [(_lib.DTYPE_BF16, _lib.KV_BF16), (_lib.DTYPE_F16, _lib.KV_F16)],
                         ids=["bf16", "f16"])
def test_prefill_causal(backend, shape, fmt):
    hq, hkv, d = shape
    _run(backend, hq, hkv, d, fmt[0], fmt[1], kv_len=[70, 33, 5], q_len=[70, 33, 5])
    _run(backend, hq, hkv, d, fmt[0], fmt[1], kv_len=[300, 17], q_len=[45, 17], chunk_pages=2, seed=1)


@pytest.mark.parametrize("q_dtype", [_lib.DTYPE_BF16, _lib.DTYPE_F16], ids=["bf16q", "f16q"])
@pytest.mark.parametrize("fmt", [_lib.KV_FP8_E4M3, _lib.KV_MXFP8], ids=["fp8", "mxfp8"])
@pytest.mark.parametrize("d", [128, 256])
def test_prefill_fp8(backend, fmt, d, q_dtype):
    """FP8 / MXFP8 pools with bf16 or f16 queries (BatchPrefillConfig.dtype
    0 = f16, 1 = bf16, flashinfer/batch_prefill.rs:23): the codes are
    dequantised to the query's type in the kernel."""
    _run(backend, 16, 4, d, q_dtype, fmt, kv_len=[200, 40], q_len=[64, 40], chunk_pages=3, seed=d + q_dtype)
    _run(backend, 32, 8, d, q_dtype, fmt, kv_len=[700], q_len=[300], causal=False, seed=d + 7 * q_dtype,
         gqa=_lib.GQA_INTERLEAVED)


@pytest.mark.parametrize("q_dtype", [_lib.DTYPE_BF16, _lib.DTYPE_F16], ids=["bf16q", "f16q"])
@pytest.mark.parametrize("fmt", [_lib.KV_FP8_E4M3, _lib.KV_MXFP8], ids=["fp8", "mxfp8"])
def test_prefill_rejects_8bit_kv_at_head_dim_64(backend, fmt, q_dtype):
    """FP8 / MXFP8 pools at head_dim 64 have no prefill kernel
    (DH_EUNSUPPORTED at plan creation, before any launch); decode takes them."""
    from dendrite_amd.backend import DhError
    with pytest.raises(DhError) as e:
        _run(backend, 16, 4, 64, q_dtype, fmt, kv_len=[40], q_len=[40])
    assert e.value.status == _lib.DH_EUNSUPPORTED


def test_prefill_chunks_gqa_invalid_and_full(backend):
    # chunk boundaries inside and across the diagonal, interleaved GQA, an
    # INVALID id in each table, and the non-causal (full) variant
    for chunk in (1, 2, 5, 0):
        _run(backend, 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, kv_len=[517, 129, 16, 1],
             q_len=[200, 129, 3, 1], chunk_pages=chunk, gqa=_lib.GQA_INTERLEAVED, invalid=True, seed=chunk)
    _run(backend, 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, kv_len=[260, 40], q_len=[31, 40], causal=False,
         chunk_pages=4, seed=9)


def test_prefill_long_context_many_items(backend):
    plan = _run(backend, 32, 8, 128, _lib.DTYPE_BF16, _lib.KV_BF16, kv_len=[2048 + 300], q_len=[300], seed=3)
    assert plan.stats()["num_items"] >= 8


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("S", [37, 300])
def test_hip_backend_prefill_matches_dense_causal_attention(dt, S):
    """HipBackend.prefill: the reference's dense causal prefill (tiled GQA);
    float32 runs as a decode over per-query virtual sequences (1e-4)."""
    g = torch.Generator().manual_seed(4)
    B, hq, hkv, d = 2, 8, 2, 64
    be = HipBackend(num_pages=16, num_kv_heads=hkv, head_dim=d)
    q = torch.randn(B, hq, S, d, generator=g).to(dt)
    k = torch.randn(B, hkv, S, d, generator=g).to(dt)
    v = torch.randn(B, hkv, S, d, generator=g).to(dt)
    cfg = AttentionConfig(hq, hkv, d)
    out = be.prefill(q, k, v, None, cfg)
    assert tuple(out.shape) == (B, hq, S, d) and out.dtype == dt
    # f64 dense causal attention on the same (bf16) inputs
    qd, kd, vd = (x.double() for x in (q, k, v))
    kd = kd.repeat(1, hq // hkv, 1, 1)
    vd = vd.repeat(1, hq // hkv, 1, 1)
    s = qd @ kd.transpose(2, 3) * cfg.scale
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    ref = torch.softmax(s, -1) @ vd
    code = _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16
    err = excess_err(out.float().cpu().numpy(), ref.numpy(), code)
    assert err <= TOL[code], err


@pytest.mark.parametrize("chunk", [1000, 5000], ids=["chunk1000", "chunk5000"])
def test_prefill_items_longer_than_decode_items(backend, chunk):
    """Items of more than 256 pages (a prefill item's page-id list holds
    2048), and a context longer than that, which the planner cuts into
    chunks whatever chunk_pages asks for."""
    _run(backend, 8, 2, 128, _lib.DTYPE_BF16, _lib.KV_BF16, kv_len=[5100, 4200], q_len=[100, 33],
         chunk_pages=chunk, seed=11)
    _run(backend, 4, 1, 128, _lib.DTYPE_BF16, _lib.KV_BF16, kv_len=[33000], q_len=[40], chunk_pages=chunk, seed=12)
    _run(backend, 8, 2, 256, _lib.DTYPE_BF16, _lib.KV_MXFP8, kv_len=[6000], q_len=[20], chunk_pages=chunk, seed=13)
