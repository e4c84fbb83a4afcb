"""Benchmark of one decode step of the paged tree-decode attention path.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3] [--no-cpu]

A step is one dh_decode_batch call (attention items + log-sum-exp merge) over
the workload's whole batch, with pages, queries and plans resident in HBM.
The default workload is c3, the Llama-3-8B-shape 64-leaf MCTS tree the
headline metric is quoted on.  To keep the 256 MB last-level cache from
serving repeats, the step rotates over several copies of the tree on disjoint
pages (more bytes than that cache holds).

Prints one JSON line (rank 0).  value = algorithmic bytes / step time, in GB/s
(algorithmic bytes: each referenced page's valid K/V bytes once, plus scale
bytes, q and out).  roofline: the attention-item kernel alone, timed with HIP
events on the stream it runs on, against the 8 TB/s HBM peak.  cpu_baseline:
the C restatement of ReferenceBackend::decode (candle op order, f32,
materialised gather/tile) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn achieved HBM GB/s (% of peak) + µs/step, 64-leaf 8B-shape tree"
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_workloads(name: str, rotations: int):
    from dendrite_amd import workloads
    if name == "c3":
        per = workloads.c3().meta["pages_per_tree"]
        rotations = max(1, min(rotations, 65536 // per))
        return [workloads.c3(rotation=r) for r in range(rotations)]
    return [workloads.ALL[name]()]


def cpu_baseline(w, budget_s: float = 12.0):
    """Times the oracle's candle-order f32 decode on a sample of sequences,
    first one thread, then all host cores; scales to a full step."""
    import oracle
    ids = w.page_ids()
    data, scales = w.make_pages(ids)
    pv = oracle.PoolView(ids, data, scales, w.num_pool_pages, w.kv_format, w.hkv, w.d)
    q = w.make_q()
    cfg = w.attention_config()
    mode = "candle" if w.name in ("c1", "c2", "c3") else "stream"
    threads = oracle.lib().oracle_num_threads()
    res = {}
    for nthr in (1, threads):
        seqs, t_used = [], 0.0
        order = np.random.Generator(np.random.PCG64(7)).permutation(w.batch)
        for b in order:
            t0 = time.perf_counter()
            oracle.decode(pv, q, w.q_dtype, w.hq, cfg.scale, w.gqa_mapping, w.indptr, w.indices,
                          w.last_page_len, seqs=[int(b)] * max(1, nthr), threads=nthr, mode=mode)
            dt = time.perf_counter() - t0
            seqs.append(int(b))
            t_used += dt
            if t_used > budget_s / 2:
                break
        # each call ran nthr copies of one sequence in parallel
        per_seq = t_used / (len(seqs) * max(1, nthr))
        step_s = per_seq * w.batch
        res[nthr] = (step_s, len(seqs) * max(1, nthr))
    step_s, nsample = res[threads]
    step1, n1 = res[1]
    return {
        "value": round(w.algorithmic_bytes() / step_s / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "us_per_step": round(step_s * 1e6, 1),
        "sample": f"{nsample} sequence decodes of {w.name} ({mode} f32, OpenMP over sequences) "
                  f"scaled to the {w.batch}-sequence step",
        "one_thread": {"value": round(w.algorithmic_bytes() / step1 / 1e9, 4), "unit": "GB/s",
                       "us_per_step": round(step1 * 1e6, 1), "sample": f"{n1} sequence decodes"},
    }


def measured_traffic(workload: str):
    """(HBM bytes per launch of the attention kernel from the committed
    rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy
    calibration), note).  The summary records a SHA-256 over the sources
    that shape the kernel's traffic; when these files differ now, the
    figure belongs to other code: bytes None, and the note says so."""
    import hashlib
    path = os.path.join(ROOT, "profiles", f"attend16_{workload}_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    h = hashlib.sha256()
    try:
        for src in t.get("sources", []):
            with open(os.path.join(ROOT, src), "rb") as f:
                h.update(f.read())
    except OSError:
        return None, "counter summary's sources not found"
    if not t.get("sources") or h.hexdigest() != t.get("sources_sha256"):
        return None, (f"stale: counters taken at {t.get('commit', '?')[:12]} on other sources "
                      f"({t.get('hbm_bytes_per_launch')} B then)")
    return t.get("hbm_bytes_per_launch"), f"counters taken at {t.get('commit', '?')[:12]} on these sources"


def warm_up(step, args) -> int:
    """Untimed calls: args.warmup of them, then more until args.warm_seconds
    of back-to-back calls have run (timed first, the first ~0.1 s of calls
    run slower than the steady state).  Returns the number of calls."""
    import torch
    t0 = time.perf_counter()
    i = 0
    while i < args.warmup or time.perf_counter() - t0 < args.warm_seconds:
        step(i)
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()     # the host clock follows the device
    torch.cuda.synchronize()
    return i


def bench_prefill(args):
    """Paged causal prefill: B sequences of CTX cached + NEW query tokens in
    shuffled pool pages; q / out [B*NEW, Hq, D] resident in HBM.  The work
    is MFMA-bound: flops = 4 Hq D sum over queries of the tokens each sees
    (QK and PV products); the roofline peak is the dense MFMA rate of the
    compute dtype."""
    import torch
    from dendrite_amd import workloads
    from dendrite_amd.backend import Backend, Pool, PrefillPlan, decode_batch
    spec, _, nb = args.prefill.partition("x")
    ctx, new = (int(x) for x in spec.split(":"))
    B = int(nb) if nb else 1
    w = workloads.ALL[args.workload]()
    kv = ctx + new
    npg = (kv + 15) // 16
    pool_pages = B * npg
    be = Backend(0)
    pool = Pool(be, pool_pages, w.hkv, w.d, w.kv_format)
    perm = np.random.default_rng(1).permutation(pool_pages).astype(np.uint32)
    ids = np.arange(pool_pages, dtype=np.uint32)
    for c0 in range(0, pool_pages, 8192):
        data, scales = w.make_pages(ids[c0:c0 + 8192])
        pool.write_pages(ids[c0:c0 + 8192], data, scales)
    indptr = np.arange(B + 1, dtype=np.uint32) * npg
    plan = PrefillPlan(be, w.attention_config(), pool, indptr, perm, np.full(B, kv, np.uint32),
                       np.full(B, new, np.uint32), causal=True)
    dt = torch.bfloat16 if w.q_dtype == 1 else torch.float16
    q = torch.randn((B * new, w.hq, w.d), device="cuda").to(dt)
    out = torch.empty_like(q)
    ws = plan.workspace()
    stream = torch.cuda.current_stream()
    warm_up(lambda i: decode_batch(plan, q, out, ws, stream=stream), args)
    res = {}
    for stages in (3, 1):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            decode_batch(plan, q, out, ws, stream=stream, stages=stages)
        e1.record(stream)
        torch.cuda.synchronize()
        res[stages] = e0.elapsed_time(e1) * 1e3 / args.steps
    seen = B * (new * ctx + new * (new + 1) // 2)
    flops = 4.0 * w.hq * w.d * seen
    tf = flops / (res[3] * 1e-6) / 1e12
    tf_att = flops / (res[1] * 1e-6) / 1e12
    peak = 2500.0   # dense bf16 / f16 MFMA, TFLOP/s
    print(json.dumps({"metric": "paged causal prefill throughput", "value": round(tf, 2), "unit": "TFLOP/s",
                      "us_per_call": round(res[3], 2), "tokens_per_s": round(B * new / (res[3] * 1e-6), 1),
                      "roofline": {"bound": "mfma", "achieved": round(tf_att, 2), "peak": peak, "unit": "TFLOP/s",
                                   "frac": round(tf_att / peak, 4), "attention_us": round(res[1], 2)},
                      "config": {"workload": w.name, "num_heads": w.hq, "num_kv_heads": w.hkv, "head_dim": w.d,
                                 "kv_format": w.kv_format, "context": ctx, "new_tokens": new, "sequences": B,
                                 "plan_items": plan.stats()["num_items"], "flops": flops},
                      "steps": args.steps, "warmup": args.warmup}), flush=True)


def bench_trait(args):
    """--trait: one decode step through HipBackend.decode_batch, the
    AttentionBackend path (host BlockTables in, the plan cached across calls
    and patched at page boundaries), on C3 with every leaf growing one token
    per step, against the raw dh_decode_batch step of one fixed plan over the
    same tables.  The new tokens' K/V are pre-written (the engine's
    append_kv is not part of the step): growth updates the tables and the
    backend's token counts only.  Each step is measured from a synchronised
    start: host time of the call, GPU span of what it enqueued (events
    around the call), and call-to-completion latency."""
    import torch
    from dendrite_amd import workloads
    from dendrite_amd.backend import DecodePlan, HipBackend, decode_batch, raw_to_tensor
    from dendrite_amd.cache import BlockTable
    w = workloads.c3()
    B, H, D = w.batch, w.hq, w.d
    total_steps = args.steps + args.warmup
    spares_n = B * (total_steps // 16 + 2)
    num_pages = w.num_pool_pages + spares_n
    be = HipBackend(num_pages=num_pages, num_kv_heads=w.hkv, head_dim=D, kv_format=w.kv_format)
    ids = np.concatenate([w.page_ids(), np.arange(w.num_pool_pages, num_pages, dtype=np.uint32)])
    for c0 in range(0, len(ids), 8192):
        data, scales = w.make_pages(ids[c0:c0 + 8192])
        be.pool.write_pages(ids[c0:c0 + 8192], data, scales)
    for p in w.page_ids():
        be.page_len[int(p)] = 16
    tables, last, pos = [], [], []
    for b in range(B):
        pages = [int(x) for x in w.seq_pages(b)]
        tables.append(BlockTable.from_blocks(pages, num_tokens=w.seq_len(b)))
        last.append(pages[-1])
        pos.append(w.seq_len(b))
        be.page_len[pages[-1]] = w.seq_len(b) - 16 * (len(pages) - 1)
    cfg = w.attention_config()
    q = raw_to_tensor(w.make_q(), w.q_dtype)
    queries = [q[i].view(1, H, 1, D) for i in range(B)]
    spare = iter(range(w.num_pool_pages, num_pages))

    def grow():
        for i, t in enumerate(tables):
            if pos[i] % 16 == 0:
                last[i] = next(spare)
                t.push(last[i])
                be.page_len[last[i]] = 1
            else:
                be.page_len[last[i]] += 1
            t.add_tokens(1)
            pos[i] += 1

    def raw_plan():
        indptr, indices, lpl = be._csr(tables)
        plan = DecodePlan(be.backend, _trait_cfg(be, cfg, q.dtype), be.pool, indptr, indices, cascade=True)
        return plan, torch.from_numpy(lpl).cuda()

    for _ in range(args.warmup):
        be.decode_batch(queries, tables, cfg)
        grow()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    host, gpu, lat = [], [], []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        be.decode_batch(queries, tables, cfg)
        ev1.record()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        host.append(t1 - t0)
        lat.append(t2 - t0)
        gpu.append(ev0.elapsed_time(ev1) * 1e-3)
        grow()
    st = dict(built=be.plans_built, patched=be.plans_patched, reused=be.plans_reused)
    # The raw step on the final tables: one fixed plan, back-to-back and
    # from a synchronised start like the trait calls.
    t0 = time.perf_counter()
    plan, lpl = raw_plan()
    plan_s = time.perf_counter() - t0
    out = torch.empty_like(q)
    ws = plan.workspace()
    for _ in range(10):
        decode_batch(plan, q, out, ws, lpl)
    torch.cuda.synchronize()
    rlat, rgpu = [], []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        decode_batch(plan, q, out, ws, lpl)
        ev1.record()
        torch.cuda.synchronize()
        rlat.append(time.perf_counter() - t0)
        rgpu.append(ev0.elapsed_time(ev1) * 1e-3)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        decode_batch(plan, q, out, ws, lpl)
    torch.cuda.synchronize()
    raw_b2b = (time.perf_counter() - t0) / args.steps
    med = lambda x: float(np.median(x)) * 1e6  # noqa: E731
    log(f"[bench] trait: host {med(host):.1f} us/call, GPU span {med(gpu):.1f} us, latency {med(lat):.1f} us; "
        f"raw: GPU span {med(rgpu):.1f} us, latency {med(rlat):.1f} us, back-to-back {raw_b2b * 1e6:.1f} us; "
        f"plans {st}; a new plan costs {plan_s * 1e6:.0f} us")
    print(json.dumps({"metric": "trait decode step (HipBackend.decode_batch, C3 growing 1 token/step)",
                      "unit": "us", "higher_is_better": False,
                      "trait_host_us_per_call": round(med(host), 2),
                      "trait_gpu_span_us": round(med(gpu), 2),
                      "trait_latency_us": round(med(lat), 2),
                      "raw_gpu_span_us": round(med(rgpu), 2),
                      "raw_latency_us": round(med(rlat), 2),
                      "raw_back_to_back_us": round(raw_b2b * 1e6, 2),
                      "new_plan_us": round(plan_s * 1e6, 1),
                      "plans": st, "steps": args.steps, "warmup": args.warmup,
                      "config": {"workload": "c3", "batch": B, "growth": "1 token per leaf per step"}}),
          flush=True)


def _trait_cfg(be, config, qdt):
    from dendrite_amd.backend import AttentionConfig, dtype_code
    cfg = AttentionConfig(config.num_heads, config.num_kv_heads, config.head_dim)
    cfg.scale = config.scale
    cfg.gqa_mapping = config.gqa_mapping
    cfg.q_dtype = dtype_code(qdt)
    cfg.kv_format = be.pool.kv_format
    return cfg


def bench_plan_timing(args):
    """Host cost of keeping a decode plan current: dh_plan_create (planning
    and upload) against dh_plan_update with one appended page for each of
    32 sequences (the events of a decode step), medians."""
    import time
    import torch
    from dendrite_amd import _lib, workloads
    from dendrite_amd.backend import Backend, DecodePlan, Pool
    be = Backend(0)
    w = workloads.ALL[args.workload]()
    pool = Pool(be, w.num_pool_pages, w.hkv, w.d, w.kv_format)
    cfg = w.attention_config()
    t_create = []
    for _ in range(7):
        t0 = time.perf_counter()
        plan = DecodePlan(be, cfg, pool, w.indptr, w.indices)
        t_create.append(time.perf_counter() - t0)
    n_ev = min(32, w.batch)
    t_update, patched = [], 0
    for k in range(16):          # 16 rounds: every sequence keeps room for its appends
        seqs = [(k * n_ev + j) % w.batch for j in range(n_ev)]
        ev = [(b, _lib.PLAN_APPEND, int(w.indices[w.indptr[b]])) for b in seqs]
        t0 = time.perf_counter()
        patched += plan.update(ev)
        t_update.append(time.perf_counter() - t0)
    torch.cuda.synchronize()
    print(json.dumps({"metric": "decode plan upkeep (host)", "workload": w.name,
                      "create_us": round(1e6 * float(np.median(t_create)), 1),
                      "update_us": round(1e6 * float(np.median(t_update)), 1),
                      "update_events": n_ev, "patched": patched, "rounds": len(t_update),
                      "note": "update through the Python binding; create includes the plan upload"}))


def bench_write(args):
    """Quantise-on-write throughput: N bf16 pages [2][Hkv][16][D] resident in
    HBM into a pool of the workload's shape and format, through
    dh_pool_write_pages_device.  Bytes per page: the bf16 source read, the
    page and its scale record written."""
    import torch
    from dendrite_amd import workloads
    from dendrite_amd.backend import Backend, Pool
    w = workloads.ALL[args.workload]()
    n = args.write_pages
    be = Backend(0)
    pool = Pool(be, n, w.hkv, w.d, w.kv_format)
    g = torch.Generator(device="cuda").manual_seed(1)
    src = torch.randn((n, 2, w.hkv, 16, w.d), generator=g, device="cuda").to(torch.bfloat16)
    ids = torch.randperm(n, device="cuda").to(torch.int32)
    stream = torch.cuda.current_stream()
    warm_up(lambda i: pool.write_pages_device(ids, src, stream=stream), args)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        pool.write_pages_device(ids, src, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    per_page = src[0].numel() * 2 + pool.page_bytes + pool.scale_bytes
    gbs = n * per_page / (us * 1e-6) / 1e9
    print(json.dumps({"metric": "quantise-on-write page throughput", "value": round(gbs, 2), "unit": "GB/s",
                      "us_per_call": round(us, 3), "pages": n, "bytes_per_page": per_page,
                      "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
                      "config": {"workload": w.name, "num_kv_heads": w.hkv, "head_dim": w.d,
                                 "kv_format": w.kv_format, "source": "bf16"},
                      "steps": args.steps, "warmup": args.warmup}), flush=True)


def bench_csr(args):
    """One decode step through dh_decode_csr (BatchDecodeKernel::run's
    contract): device int32 CSR tables read on the GPU every call, no plan.
    The decomposition is flat, so shared pages are streamed once per
    sequence: the rate is given against the workload's unique bytes (the
    metric of the planned path) and against the bytes this path reads."""
    import torch
    from dendrite_amd import _lib
    from dendrite_amd.backend import Backend, Pool, csr_workspace_size, decode_csr, raw_to_tensor
    w = workloads_one(args.workload)
    be = Backend(0)
    pool = Pool(be, w.num_pool_pages, w.hkv, w.d, w.kv_format)
    ids = w.page_ids()
    for c0 in range(0, len(ids), 8192):
        data, scales = w.make_pages(ids[c0:c0 + 8192])
        pool.write_pages(ids[c0:c0 + 8192], data, scales)
        del data, scales
    cfg = w.attention_config()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).cuda()  # noqa: E731
    ix, ip, lp = dev(w.indices), dev(w.indptr), dev(w.last_page_len)
    q = raw_to_tensor(w.make_q(), w.q_dtype)
    out = torch.empty_like(q)
    ws = torch.empty(csr_workspace_size(cfg, w.batch, int(w.indptr[-1])), dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def step(i):
        decode_csr(be, pool, cfg, q, ix, ip, lp, out, ws, status, stream=stream)

    warm_up(step, args)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    if int(status.item()) != 0:
        raise RuntimeError(f"dh_decode_csr status {int(status.item())}")
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    alg = w.algorithmic_bytes()
    qo = 2 * w.batch * w.hq * w.d * (4 if w.q_dtype == _lib.DTYPE_F32 else 2)
    streamed = w.naive_kv_bytes() + qo
    if w.kv_format == _lib.KV_MXFP8:        # one scale byte per 32 values
        streamed += w.naive_kv_bytes() // 32
    unique_gbs = alg / (us * 1e-6) / 1e9
    streamed_gbs = streamed / (us * 1e-6) / 1e9
    log(f"[bench] csr {w.name}: {us:.2f} us/step, {unique_gbs:.0f} GB/s of unique bytes, "
        f"{streamed_gbs:.0f} GB/s of streamed bytes")
    print(json.dumps({"metric": "paged decode step from device CSR (dh_decode_csr)", "value": round(us, 2),
                      "unit": "us", "higher_is_better": False,
                      "unique_bytes": alg, "unique_gbs": round(unique_gbs, 1),
                      "streamed_bytes": streamed, "streamed_gbs": round(streamed_gbs, 1),
                      "streamed_pct_of_peak_hbm": round(100 * streamed_gbs / PEAK_HBM_GBS, 2),
                      "config": {"workload": w.name, "batch": w.batch, "num_heads": w.hq,
                                 "num_kv_heads": w.hkv, "head_dim": w.d, "kv_format": w.kv_format},
                      "steps": args.steps, "warmup": args.warmup}), flush=True)


def workloads_one(name: str):
    from dendrite_amd import workloads
    return workloads.ALL[name]()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c3")
    ap.add_argument("--rotations", type=int, default=6)
    ap.add_argument("--warm-seconds", type=float, default=0.25,
                    help="untimed steps continue after --warmup until this much time has passed")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--shared-chunk", type=int, default=0)
    ap.add_argument("--private-chunk", type=int, default=0)
    ap.add_argument("--target-items", type=int, default=0)
    ap.add_argument("--flat", action="store_true", help="plan option: no cascade (every sequence alone)")
    ap.add_argument("--no-direct", action="store_true", help="plan option: never a direct (merge-free) plan")
    ap.add_argument("--trait", action="store_true",
                    help="only measure the AttentionBackend path (HipBackend.decode_batch) on C3 with tables "
                         "growing one token per step, against the raw step")
    ap.add_argument("--plan-timing", action="store_true",
                    help="only time dh_plan_create against dh_plan_update (32 appended pages) on the host")
    ap.add_argument("--prefill", default="", metavar="CTX:NEW[xB]",
                    help="only measure paged causal prefill: NEW query tokens after CTX cached tokens, "
                         "B sequences, at the workload's head shape and KV format (e.g. 0:4096, 8192:2048x4)")
    ap.add_argument("--write-pages", type=int, default=0, metavar="N",
                    help="only measure quantise-on-write (dh_pool_write_pages_device) of N bf16 pages "
                         "into a pool of the workload's shape and KV format")
    ap.add_argument("--csr", action="store_true",
                    help="only measure dh_decode_csr (device CSR tables, no plan) on the workload")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB five times (the known-size "
                         "kernel that scales the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (across GPUs "
                                   "the path would shard by tree or by KV head, with no kernel change)"}))
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return

    from dendrite_amd.backend import Backend, DecodePlan, Pool, decode_batch, raw_to_tensor

    if args.trait:
        bench_trait(args)
        return
    if args.plan_timing:
        bench_plan_timing(args)
        return
    if args.write_pages:
        bench_write(args)
        return
    if args.prefill:
        bench_prefill(args)
        return
    if args.csr:
        bench_csr(args)
        return

    ws_list = build_workloads(args.workload, args.rotations)
    w0 = ws_list[0]
    log(f"[bench] workload {w0.name}: {w0.description}; {len(ws_list)} rotation(s)")
    be = Backend(0)
    pool = Pool(be, w0.num_pool_pages, w0.hkv, w0.d, w0.kv_format)
    plans, qs, outs, lpls = [], [], [], []
    for w in ws_list:
        ids = w.page_ids()
        # Synthesised and uploaded in chunks: bounded host memory, and a
        # progress line per chunk for the multi-GB configs (C4, C5).
        chunk = 8192
        for c0 in range(0, len(ids), chunk):
            data, scales = w.make_pages(ids[c0:c0 + chunk])
            pool.write_pages(ids[c0:c0 + chunk], data, scales)
            del data, scales
            if len(ids) > chunk:
                log(f"[bench] pages {min(c0 + chunk, len(ids))}/{len(ids)} written")
        plan = DecodePlan(be, w.attention_config(), pool, w.indptr, w.indices, cascade=not args.flat,
                          shared_chunk_pages=args.shared_chunk,
                          private_chunk_pages=args.private_chunk, target_items=args.target_items,
                          direct=not args.no_direct)
        plans.append(plan)
        q = raw_to_tensor(w.make_q(), w.q_dtype)
        qs.append(q)
        outs.append(torch.empty_like(q))
        lpls.append(torch.from_numpy(np.ascontiguousarray(w.last_page_len)).cuda())
    ws = torch.empty(max(p.workspace_size for p in plans) + 256, dtype=torch.uint8, device="cuda")
    st = plans[0].stats()
    log(f"[bench] plan: {st}")
    alg = w0.algorithmic_bytes()
    alg_attend = alg - w0.batch * w0.hq * w0.d * (4 if w0.q_dtype == 2 else 2)   # no O writes
    stream = torch.cuda.current_stream()
    R = len(plans)

    def step(i, stages=3):
        k = i % R
        decode_batch(plans[k], qs[k], outs[k], ws, lpls[k], stream=stream, stages=stages)

    # Warm-up (warm_up): C5 timed without it 898 against 797 us a step, C4
    # 233 against 223, whatever the step count.
    t_warm = time.perf_counter()
    n_warm = warm_up(step, args)
    log(f"[bench] warm-up: {n_warm} steps in {time.perf_counter() - t_warm:.2f} s")

    def timed(stages):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record(stream)
        for i in range(args.steps):
            step(i, stages)
        ev1.record(stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / args.steps

    ms_step = timed(3)
    ms_attend = timed(1)
    ms_merge = timed(2)
    # per-step distribution (single-step event pairs)
    per = []
    for i in range(min(args.steps, 100)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        step(i)
        e1.record(stream)
        e1.synchronize()
        per.append(e0.elapsed_time(e1))
    per = np.array(per)
    log(f"[bench] step {ms_step * 1e3:.2f} us (attend {ms_attend * 1e3:.2f} us, merge {ms_merge * 1e3:.2f} us)"
        f"; single-step median {np.median(per) * 1e3:.2f} us")

    traffic, traffic_note = measured_traffic(w0.name)
    gbs = alg / (ms_step * 1e-3) / 1e9
    attend_gbs = alg_attend / (ms_attend * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": n_warm,
        "ms_per_step": round(ms_step, 6),
        "us_per_step": round(ms_step * 1e3, 3),
        "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "tokens_per_s": round(w0.batch / (ms_step * 1e-3), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {1: "bf16", 0: "f16", 2: "f32"}[w0.q_dtype] +
                 ({3: "+fp8e4m3-kv", 4: "+mxfp8-kv"}.get(w0.kv_format, "")),
        "data": "synthetic (seeded N(0,1) K/V/q; tree shape per config)",
        "config": {
            "workload": f"{w0.name}: {w0.description}",
            "leaves": w0.batch, "num_heads": w0.hq, "num_kv_heads": w0.hkv, "head_dim": w0.d,
            "algorithmic_bytes_per_step": alg, "flops_per_step": w0.flops(),
            "unique_pages": st["unique_pages"], "page_reads_per_kv_head": st["page_reads"],
            "naive_kv_bytes": w0.naive_kv_bytes(), "rotations": R, "plan_items": st["num_items"],
            "partials_per_row": st["num_partials"] / max(1, w0.batch),
        },
        "single_step_us": {"p10": round(float(np.percentile(per, 10)) * 1e3, 2),
                           "median": round(float(np.median(per)) * 1e3, 2),
                           "p90": round(float(np.percentile(per, 90)) * 1e3, 2)},
        "roofline": {
            "bound": "hbm",
            "kernel": "attend16_kernel (attention items)",
            "achieved": round(attend_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(attend_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_note": traffic_note,
            "avg_launch_us": round(ms_attend * 1e3, 3),
            "merge_launch_us": round(ms_merge * 1e3, 3),
            "mfma_tflops": round(w0.flops() / (ms_attend * 1e-3) / 1e12, 2),
        },
    }
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(w0)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
