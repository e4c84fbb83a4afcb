"""Randomised parity sweep: seeded random fork trees over every head shape and
dtype / format pair, with random plan options (cascade or flat, chunk sizes,
direct plans on or off), GQA mappings and softmax scales, through the plan
path (dh_decode_batch) and the device-CSR path (dh_decode_csr), and random
prefill batches, each case against the CPU oracle on the same inputs.  The cases are fixed by the seeds,
so a failure names a reproducible case (printed before it runs)."""
import numpy as np
import pytest

import oracle
from dendrite_amd import _lib, workloads
from dendrite_amd.backend import Pool, csr_workspace_size, decode_csr
from tests._helpers import TOL, GpuRun, excess_err, max_abs_err, q_tensor

pytestmark = pytest.mark.gpu

SHAPES = [(32, 4, 64), (32, 8, 128), (16, 2, 256), (64, 8, 128), (64, 2, 128), (32, 1, 64), (8, 8, 128),
          (128, 2, 128)]
FMTS = [(_lib.DTYPE_BF16, _lib.KV_BF16), (_lib.DTYPE_F16, _lib.KV_F16), (_lib.DTYPE_F32, _lib.KV_F32),
        (_lib.DTYPE_BF16, _lib.KV_FP8_E4M3), (_lib.DTYPE_BF16, _lib.KV_MXFP8),
        (_lib.DTYPE_F16, _lib.KV_FP8_E4M3), (_lib.DTYPE_F16, _lib.KV_MXFP8)]


def _case(i, seed0):
    rng = np.random.default_rng([seed0, i])
    shape = SHAPES[rng.integers(len(SHAPES))]
    fmt = FMTS[rng.integers(len(FMTS))]
    tree = dict(n_leaves=int(rng.integers(1, 40)), max_run=int(rng.choice([3, 9, 20, 40, 80])),
                pool_pages=4096, partial=bool(rng.random() < 0.7))
    seed = int(rng.integers(1 << 30))
    gqa = _lib.GQA_INTERLEAVED if rng.random() < 0.3 else _lib.GQA_TILED
    plan = {}
    if rng.random() < 0.3:
        plan["shared_chunk_pages"] = int(rng.choice([1, 2, 8, 16, 64]))
    if rng.random() < 0.3:
        plan["private_chunk_pages"] = int(rng.choice([1, 2, 8, 16, 64]))
    if rng.random() < 0.2:
        plan["direct"] = False
    cascade = bool(rng.random() < 0.6)
    scale = float(rng.choice([0.0, -0.3, 1.5, 0.05])) if rng.random() < 0.2 else None
    return shape, fmt, tree, seed, gqa, plan, cascade, scale


@pytest.mark.parametrize("i", range(48))
def test_random_plan_decode(backend, i):
    shape, fmt, tree, seed, gqa, plan, cascade, scale = _case(i, 0x5EED)
    w = workloads.random_tree(seed, *shape, fmt[0], fmt[1], **tree)
    w.gqa_mapping = gqa
    print(f"[case] sweep {i}: shape {shape} fmt {fmt} tree {tree} seed {seed} gqa {gqa} cascade {cascade} "
          f"plan {plan} scale {scale}", flush=True)
    run = GpuRun(w, backend, cascade=cascade, scale=scale, **plan)
    got, ref = run.run(), run.reference()
    err = excess_err(got, ref, w.q_dtype)
    print(f"[case] sweep {i}: max abs err {max_abs_err(got, ref):.3e}, beyond output rounding {err:.3e}", flush=True)
    assert np.all(np.isfinite(got)) and err <= TOL[w.q_dtype]


@pytest.mark.parametrize("i", range(24))
def test_random_csr_decode(backend, i):
    import torch
    shape, fmt, tree, seed, _, _, _, _ = _case(i, 0xC5A)
    w = workloads.random_tree(seed, *shape, fmt[0], fmt[1], **tree)
    print(f"[case] csr sweep {i}: shape {shape} fmt {fmt} tree {tree} seed {seed}", flush=True)
    pool = Pool(backend, w.num_pool_pages, w.hkv, w.d, w.kv_format)
    ids = w.page_ids()
    data, scales = w.make_pages(ids)
    pool.write_pages(ids, data, scales)
    cfg = w.attention_config()
    q_raw = w.make_q()
    q = q_tensor(q_raw, w.q_dtype)
    out = torch.full_like(q, float("nan"))
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda:0")
    ws = torch.empty(csr_workspace_size(cfg, w.batch, max(1, int(w.indptr[-1]))), dtype=torch.uint8,
                     device="cuda:0")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to("cuda:0")  # noqa: E731
    ix = dev(w.indices if len(w.indices) else np.zeros(1, np.int32))
    decode_csr(backend, pool, cfg, q, ix, dev(w.indptr), dev(w.last_page_len), out, ws, status)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    pv = oracle.PoolView(ids, data, scales, pool.num_pages, w.kv_format, w.hkv, w.d)
    ref = oracle.decode(pv, q_raw, w.q_dtype, w.hq, cfg.scale, w.gqa_mapping, w.indptr, w.indices,
                        w.last_page_len)
    err = excess_err(got, ref, w.q_dtype)
    print(f"[case] csr sweep {i}: max abs err {max_abs_err(got, ref):.3e}, beyond output rounding {err:.3e}",
          flush=True)
    assert int(status.item()) == _lib.DH_OK
    assert np.all(np.isfinite(got)) and err <= TOL[w.q_dtype]


PREFILL_SHAPES = [(32, 8, 128), (16, 4, 64), (8, 2, 256), (32, 4, 64), (64, 8, 128)]
PREFILL_FMTS = [(_lib.DTYPE_BF16, _lib.KV_BF16), (_lib.DTYPE_F16, _lib.KV_F16),
                (_lib.DTYPE_BF16, _lib.KV_FP8_E4M3), (_lib.DTYPE_BF16, _lib.KV_MXFP8)]


@pytest.mark.parametrize("i", range(24))
def test_random_prefill(backend, i):
    """Paged prefill: random batches of (context, new tokens), causal or
    full, chunk sizes, GQA mappings and INVALID ids, against the oracle's
    decode of each query's virtual sequence (tests/test_gpu_prefill.py)."""
    from tests.test_gpu_prefill import _run
    rng = np.random.default_rng([0x9F, i])
    hq, hkv, d = PREFILL_SHAPES[rng.integers(len(PREFILL_SHAPES))]
    fmt = PREFILL_FMTS[rng.integers(len(PREFILL_FMTS))]
    if fmt[1] in (_lib.KV_FP8_E4M3, _lib.KV_MXFP8) and d == 64:
        d = 128
    B = int(rng.integers(1, 4))
    kv = [int(rng.integers(1, 600)) for _ in range(B)]
    q = [int(rng.integers(1, min(k, 64) + 1)) for k in kv]
    _run(backend, hq, hkv, d, fmt[0], fmt[1], kv_len=kv, q_len=q, causal=bool(rng.random() < 0.8),
         chunk_pages=int(rng.choice([0, 0, 1, 3, 8])),
         gqa=_lib.GQA_INTERLEAVED if rng.random() < 0.3 else _lib.GQA_TILED,
         invalid=bool(rng.random() < 0.3), seed=int(rng.integers(1 << 20)))
