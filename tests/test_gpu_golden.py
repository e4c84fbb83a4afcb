"""GPU parity against the committed golden fixtures (tests/golden/
decode_cases.npz, made by tests/golden/make_golden.py from torch's CPU
attention in f64), and known-answer tests that pin page selection
bit-exactly, all through the C ABI.

Tolerances: f32 1e-4 max-abs; bf16 / f16 / FP8 / MXFP8 2e-2 max-abs beyond
the output dtype's own rounding (tests/_helpers.excess_err).
"""
import os

import numpy as np
import pytest

from dendrite_amd import _lib
from dendrite_amd.backend import AttentionConfig, DecodePlan, Pool, decode_batch, raw_to_tensor
from tests._helpers import TOL, excess_err

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "decode_cases.npz")


def _cases():
    z = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in z.files})
    return {n: {k.split("/")[1]: z[k] for k in z.files if k.startswith(n + "/")} for n in names}


CASES = _cases()


def _decode(backend, hq, hkv, d, q_dtype, fmt, gqa, pool_pages, ids, data, scales, indptr, indices, lpl,
            q_raw, cascade=True):
    import torch
    pool = Pool(backend, pool_pages, hkv, d, fmt)
    pool.write_pages(ids, data, scales if scales is not None and scales.size else None)
    cfg = AttentionConfig(hq, hkv, d)
    cfg.q_dtype, cfg.kv_format, cfg.gqa_mapping = q_dtype, fmt, gqa
    plan = DecodePlan(backend, cfg, pool, indptr, indices, cascade=cascade)
    B = len(indptr) - 1
    q = raw_to_tensor(np.ascontiguousarray(q_raw).reshape(B, -1), q_dtype).reshape(B, hq, d)
    out = torch.full_like(q, float("nan"))
    lp = torch.from_numpy(np.ascontiguousarray(lpl, dtype=np.int32)).cuda()
    decode_batch(plan, q, out, plan.workspace(), lp)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("cascade", [True, False])
@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_case(backend, name, cascade):
    c = CASES[name]
    hq, hkv, d, q_dtype, fmt, gqa, pool_pages = (int(x) for x in c["meta"])
    print(f"[case] golden {name} cascade={cascade}", flush=True)
    got = _decode(backend, hq, hkv, d, q_dtype, fmt, gqa, pool_pages, c["ids"], c["data"], c["scales"],
                  c["indptr"], c["indices"], c["last_page_len"], c["q"], cascade)
    assert np.all(np.isfinite(got))
    err = excess_err(got, c["out"], q_dtype)
    print(f"[case] golden {name}: beyond-rounding error {err:.3e}", flush=True)
    assert err <= TOL[q_dtype]


def test_golden_empty_sequence_is_exact_zero(backend):
    c = CASES["bf16_tree"]
    hq, hkv, d, q_dtype, fmt, gqa, pool_pages = (int(x) for x in c["meta"])
    got = _decode(backend, hq, hkv, d, q_dtype, fmt, gqa, pool_pages, c["ids"], c["data"], c["scales"],
                  c["indptr"], c["indices"], c["last_page_len"], c["q"])
    assert not np.any(got[3])


def test_golden_single_token_is_exact_v_row(backend):
    c = CASES["f32_one_token"]
    hq, hkv, d, q_dtype, fmt, gqa, pool_pages = (int(x) for x in c["meta"])
    got = _decode(backend, hq, hkv, d, q_dtype, fmt, gqa, pool_pages, c["ids"], c["data"], c["scales"],
                  c["indptr"], c["indices"], c["last_page_len"], c["q"])
    v = c["data"][0].view(np.float32).reshape(2, hkv, 16, d)[1, :, 0]
    for h in range(hq):
        assert np.array_equal(got[0, h], v[h % hkv])


@pytest.mark.parametrize("kvf", [_lib.KV_BF16, _lib.KV_F32])
@pytest.mark.parametrize("gqa", [_lib.GQA_TILED, _lib.GQA_INTERLEAVED])
def test_one_hot_selects_exact_v_row(backend, kvf, gqa):
    """V rows hold small integers that encode (page, slot, head); each query
    head's logit on one chosen token beats every other by 181 nats (2^-261:
    every other weight underflows to exactly 0 in f32), so the output must
    equal that V row bit for bit.  A wrong page,
    slot, plane, head or GQA index reads a different integer.  Sequences share
    prefixes (cascade items), and the target sits in shared and private pages
    and past a partial last page's valid tokens (a larger logit there must be
    ignored)."""
    hq, hkv, d = 16, 4, 128
    r = hq // hkv
    rng = np.random.Generator(np.random.PCG64(17 + kvf + 3 * gqa))
    pool_pages = 64
    perm = [int(x) for x in rng.permutation(pool_pages)]
    prefix = perm[:6]
    tables = [prefix + perm[6 + 3 * i:9 + 3 * i] for i in range(5)]     # 9 pages each
    lpl = np.array([16, 5, 9, 1, 12], dtype=np.int32)
    ids = sorted({p for t in tables for p in t})
    # V integers stay exact in bf16 (8 significant bits): (page index in ids,
    # slot, head) go to three separate dims.
    pages = {}
    for k, pid in enumerate(ids):
        p = pages[pid] = np.zeros((2, hkv, 16, d), dtype=np.float32)
        for h in range(hkv):
            for s in range(16):
                p[1, h, s, 0] = k
                p[1, h, s, 1] = s
                p[1, h, s, 2] = h
                p[1, h, s, 3:] = (k + s + h) % 7
    B = len(tables)
    q = np.zeros((B, hq, d), dtype=np.float32)
    want = np.zeros((B, hq, d), dtype=np.float32)
    for b, t in enumerate(tables):
        for qh in range(hq):
            kh = qh % hkv if gqa == _lib.GQA_TILED else qh // r
            j = (b * 5 + qh * 3) % len(t)
            valid = lpl[b] if j == len(t) - 1 else 16
            slot = (b + 7 * qh) % valid
            pid = t[j]
            dim = b * hq + qh                            # one q dim per (sequence, head)
            q[b, qh, dim] = 128.0
            pages[pid][0, kh, slot, dim] = 16.0          # logit 2048 * scale 0.0884 = 181 nats
            want[b, qh] = pages[pid][1, kh, slot]
            if valid < 16:                               # a larger logit past the valid tokens
                pages[t[-1]][0, kh, 15, dim] = 32.0
    # every other token scores 0 for (b, qh): keys planted for other pairs sit
    # in other dims
    if kvf == _lib.KV_BF16:
        import torch
        raw = {p: torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy() for p, v in pages.items()}
        q_raw = torch.from_numpy(q).to(torch.bfloat16).view(torch.int16).numpy()
        qd = _lib.DTYPE_BF16
    else:
        raw = pages
        q_raw = q
        qd = _lib.DTYPE_F32
    data = np.stack([raw[p].reshape(-1).view(np.uint8) for p in ids])
    indptr = np.array([0] + list(np.cumsum([len(t) for t in tables])), dtype=np.uint32)
    indices = np.array([p for t in tables for p in t], dtype=np.uint32)
    for cascade in (True, False):
        print(f"[case] one-hot kvf={kvf} gqa={gqa} cascade={cascade}", flush=True)
        got = _decode(backend, hq, hkv, d, qd, kvf, gqa, pool_pages, np.array(ids, dtype=np.uint32), data,
                      None, indptr, indices, lpl, q_raw, cascade)
        assert np.array_equal(got, want), f"max diff {np.max(np.abs(got - want))}"


@pytest.mark.parametrize("kvf", [_lib.KV_BF16, _lib.KV_FP8_E4M3, _lib.KV_MXFP8, _lib.KV_F32])
def test_gather_debug_is_byte_exact(backend, kvf):
    """dh_gather_debug reads pages with the kernels' addressing; its bytes must
    equal the host's own slice of the written pages, INVALID entries skipped."""
    from dendrite_amd import workloads
    w = workloads.random_tree(3, 16, 4, 128, _lib.DTYPE_BF16 if kvf != _lib.KV_F32 else _lib.DTYPE_F32,
                              kvf, n_leaves=4, pool_pages=256)
    pool = Pool(backend, w.num_pool_pages, w.hkv, w.d, kvf)
    ids = w.page_ids()
    data, scales = w.make_pages(ids)
    pool.write_pages(ids, data, scales)
    eb = pool.page_bytes // (2 * w.hkv * 16 * w.d)
    sel = [int(ids[5]), _lib.INVALID_PAGE, int(ids[0]), int(ids[-1]), int(ids[5])]
    row = {int(p): i for i, p in enumerate(ids)}
    for h in range(w.hkv):
        got, n = pool.gather(sel, h)
        kept = [p for p in sel if p != _lib.INVALID_PAGE]
        assert n == len(kept)
        blk = 16 * w.d * eb
        planes = [data[row[p]].reshape(2, w.hkv, blk)[:, h] for p in kept]
        want = np.concatenate([np.concatenate([pl[0] for pl in planes]),
                               np.concatenate([pl[1] for pl in planes])])
        assert np.array_equal(got, want)
