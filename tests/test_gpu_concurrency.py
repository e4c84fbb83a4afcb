"""Concurrent decode calls on one backend handle.

The reference's AttentionBackend is Send + Sync (attention/backend.rs:62): one
backend may serve several threads at once.  Here two host threads share one
dh_backend and one pool and call dh_decode_batch at the same time (ctypes
releases the GIL for the call), each with its own plan, stream, workspace and
output; every result must equal the serial result bit for bit and match the
CPU oracle.
"""
import threading

import numpy as np
import pytest

from dendrite_amd import workloads
from dendrite_amd.backend import DecodePlan, decode_batch
from tests._helpers import TOL, GpuRun, excess_err, max_abs_err, q_tensor

pytestmark = pytest.mark.gpu


def test_two_threads_share_one_backend(backend):
    import torch

    # One pool holds both workloads' pages: a tree (group items + tails) and
    # a flat batch (wave items only), same head shape and format.
    w_a = workloads.c3(root_pages=40, levels=2, level_pages=3, pool_pages=4096)
    run = GpuRun(w_a, backend)
    tables = [[int(p) for p in w_a.seq_pages(b)][-9:] for b in range(w_a.batch)]
    w_b = workloads.custom(tables, w_a.hq, w_a.hkv, w_a.d, w_a.q_dtype, w_a.kv_format, w_a.num_pool_pages,
                           last_page_len=[(5 * b) % 16 + 1 for b in range(len(tables))], seed=w_a.seed,
                           name="flat")
    cfg = run.cfg
    jobs = []
    for w, cascade in ((w_a, True), (w_b, False)):
        plan = DecodePlan(backend, cfg, run.pool, w.indptr, w.indices, cascade=cascade)
        q_raw = w.make_q()
        q = q_tensor(q_raw, w.q_dtype)
        lpl = torch.from_numpy(np.ascontiguousarray(w.last_page_len, dtype=np.int32)).to("cuda:0")
        ref = run.reference() if w is w_a else None
        if ref is None:
            import oracle
            ref = oracle.decode(run.pool_view(), q_raw, w.q_dtype, w.hq, cfg.scale, w.gqa_mapping, w.indptr,
                                w.indices, w.last_page_len)
        jobs.append(dict(w=w, plan=plan, q=q, lpl=lpl, ref=ref, ws=plan.workspace(),
                         out=torch.empty_like(q), stream=torch.cuda.Stream()))

    # Serial results first.
    for j in jobs:
        decode_batch(j["plan"], j["q"], j["out"], j["ws"], j["lpl"], stream=j["stream"])
    torch.cuda.synchronize()
    for j in jobs:
        j["serial"] = j["out"].clone()
        got = j["serial"].float().cpu().numpy()
        raw, err = max_abs_err(got, j["ref"]), excess_err(got, j["ref"], j["w"].q_dtype)
        print(f"[case] {j['w'].name} serial: max abs err {raw:.3e}, beyond output rounding {err:.3e}", flush=True)
        assert err <= TOL[j["w"].q_dtype]

    iters = 50
    start = threading.Barrier(len(jobs))
    errors = []

    def worker(j):
        try:
            start.wait()
            with torch.cuda.stream(j["stream"]):
                for _ in range(iters):
                    j["out"].fill_(float("nan"))   # no stale result can pass
                    decode_batch(j["plan"], j["q"], j["out"], j["ws"], j["lpl"], stream=j["stream"])
                    j["stream"].synchronize()
                    if not torch.equal(j["out"], j["serial"]):
                        errors.append(f"{j['w'].name}: concurrent result differs from the serial one")
                        return
        except Exception as e:   # reported by the main thread
            errors.append(f"{j['w'].name}: {e!r}")

    threads = [threading.Thread(target=worker, args=(j,)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a decode thread did not finish"
    assert not errors, errors
    print(f"[case] {len(jobs)} threads x {iters} concurrent decode calls: equal to the serial results", flush=True)


def test_two_threads_share_one_hip_backend():
    """HipBackend.decode_batch from two host threads at once, each on its own
    stream, with tables that grow one token per step (so the cached plans
    are reused, patched at page boundaries and rebuilt when the other
    thread's appends change the set of stored blocks).  The calls are not
    synchronised between steps: each stream's queued decodes overlap the
    other's.  Every step of both threads must match the oracle on the
    tables as they were at that step."""
    import torch

    from dendrite_amd import _lib
    from dendrite_amd.backend import AttentionConfig, HipBackend
    from dendrite_amd.cache import BlockTable

    hq, hkv, d, steps = 16, 4, 64, 24
    be = HipBackend(num_pages=512, num_kv_heads=hkv, head_dim=d)
    cfg = AttentionConfig(hq, hkv, d)

    def randn(shape, seed):
        g = torch.Generator().manual_seed(seed)
        return torch.randn(*shape, generator=g, dtype=torch.float32)

    prefix = [1, 2, 3]
    for i, b in enumerate(prefix):
        be.append_kv(randn((1, hkv, 16, d), 10 + 2 * i), randn((1, hkv, 16, d), 11 + 2 * i),
                     BlockTable.from_blocks([b]), 0)
    jobs = []
    for j, first in enumerate((10, 200)):
        tables, pos = [], []
        for leaf in range(4):
            n0 = 3 + 4 * leaf + j
            t = BlockTable.from_blocks(prefix + [first + leaf], num_tokens=48 + n0)
            be.append_kv(randn((1, hkv, n0, d), 1000 * (j + 1) + leaf), randn((1, hkv, n0, d), 1000 * (j + 1) + 50 + leaf),
                         t, 48)
            tables.append(t)
            pos.append(48 + n0)
        q = randn((4, hq, d), 77 + j).to(torch.bfloat16).cuda()
        jobs.append(dict(tables=tables, pos=pos, nxt=first + 4 + 100 * j, seed=5000 * (j + 1),
                         queries=[q[i].view(1, hq, 1, d) for i in range(4)], outs=[], snaps=[],
                         stream=torch.cuda.Stream()))
    torch.cuda.synchronize()
    start = threading.Barrier(len(jobs))
    errors = []

    def worker(job):
        try:
            start.wait()
            with torch.cuda.stream(job["stream"]):
                for _ in range(steps):
                    job["outs"].append(be.decode_batch(job["queries"], job["tables"], cfg))
                    job["snaps"].append(be._csr(job["tables"]))
                    for i, t in enumerate(job["tables"]):
                        if job["pos"][i] % 16 == 0:
                            t.push(job["nxt"])
                            job["nxt"] += 1
                        job["seed"] += 2
                        be.append_kv(randn((1, hkv, 1, d), job["seed"]), randn((1, hkv, 1, d), job["seed"] + 1),
                                     t, job["pos"][i])
                        t.add_tokens(1)
                        job["pos"][i] += 1
        except Exception as e:   # reported by the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(j,)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a decode thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors
    # Oracle per step: the pool as it is now holds every step's tokens (pages
    # only gained tokens past each step's lengths).
    ids = sorted({int(p) for job in jobs for snap in job["snaps"] for p in snap[1]})
    pv = oracle_pool(be, ids)
    worst = 0.0
    for j, job in enumerate(jobs):
        q = np.stack([x.reshape(hq, d).float().cpu().numpy() for x in job["queries"]])
        for s, (out, (indptr, indices, lpl)) in enumerate(zip(job["outs"], job["snaps"])):
            import oracle
            want = oracle.decode(pv, q, _lib.DTYPE_F32, hq, cfg.scale, cfg.gqa_mapping, indptr, indices, lpl)
            got = out.float().cpu().reshape(4, hq, d).numpy()
            err = float(np.max(np.abs(got - want)))
            worst = max(worst, err)
            assert err < 2e-2, (j, s, err)
    print(f"[case] 2 threads x {steps} trait steps on their own streams: max abs err {worst:.3e}; "
          f"plans built {be.plans_built}, patched {be.plans_patched}, reused {be.plans_reused}", flush=True)
    assert be.plans_patched > 0


def oracle_pool(be, ids):
    import oracle
    data = np.stack([be.pool.read_page(p)[0] for p in ids])
    return oracle.PoolView(np.array(ids, dtype=np.uint32), data, None, be.pool.num_pages, be.pool.kv_format,
                           be.pool.num_kv_heads, be.pool.head_dim)
