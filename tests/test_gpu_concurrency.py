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
