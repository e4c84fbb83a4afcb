"""dh_decode_csr: decode from device-resident int32 CSR page tables, read on
the device on every call (BatchDecodeKernel::run's contract,
crates/dendrite-ffi/src/flashinfer/batch_decode.rs:86-95), against the CPU
oracle on identical inputs, plus its error reporting: bad page ids and
indptr entries (status DH_EINVAL, zeros for those sequences, no read outside
the pool) and tables larger than the workspace (DH_ENOMEM, zeros).  Shared
prefixes of consecutive sequences (what TreeState::fork produces) are read
once per KV head by group items (CascadeAttention's promise,
crates/dendrite-ffi/src/flashinfer/cascade.rs:22-26): the call's header
records how many, and the tests below check both the grouping and the
results.
Tolerances as in test_gpu_decode (f32 1e-4; 16-bit / FP8 2e-2 beyond the
output dtype's rounding)."""
import numpy as np
import pytest

import oracle
from dendrite_amd import _lib, workloads
from dendrite_amd.backend import DhError, Pool, csr_workspace_size, decode_csr
from tests._helpers import TOL, excess_err, max_abs_err, q_tensor

pytestmark = pytest.mark.gpu


class CsrRun:
    """A workload's pages in a pool, its tables as device int32 CSR."""

    def __init__(self, w, backend, pool_pages=None, ws_pages=None):
        import torch
        self.w = w
        self.backend = backend
        self.pool = Pool(backend, pool_pages or w.num_pool_pages, w.hkv, w.d, w.kv_format)
        self.ids = w.page_ids()
        self.data, self.scales = w.make_pages(self.ids)
        self.pool.write_pages(self.ids, self.data, self.scales)
        self.cfg = w.attention_config()
        self.q_raw = w.make_q()
        self.q = q_tensor(self.q_raw, w.q_dtype)
        self.out = torch.empty_like(self.q)
        self.status = torch.full((1,), -1, dtype=torch.int32, device="cuda:0")
        total = int(w.indptr[-1]) if ws_pages is None else ws_pages
        self.ws = torch.empty(csr_workspace_size(self.cfg, w.batch, total), dtype=torch.uint8, device="cuda:0")

    def tables(self, indptr=None, indices=None, lpl=None):
        import torch
        w = self.w
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to("cuda:0")  # noqa: E731
        return (dev(w.indices if indices is None else indices), dev(w.indptr if indptr is None else indptr),
                dev(w.last_page_len if lpl is None else lpl))

    def run(self, indptr=None, indices=None, lpl=None, use_lpl=True):
        import torch
        ix, ip, lp = self.tables(indptr, indices, lpl)
        self.out.fill_(float("nan"))
        decode_csr(self.backend, self.pool, self.cfg, self.q, ix, ip, lp if use_lpl else None, self.out, self.ws,
                   self.status)
        torch.cuda.synchronize()
        return self.out.float().cpu().numpy(), int(self.status.item())

    def reference(self, seqs=None, indptr=None, indices=None, lpl=None):
        w = self.w
        pv = oracle.PoolView(self.ids, self.data, self.scales, self.pool.num_pages, w.kv_format, w.hkv, w.d)
        return oracle.decode(pv, self.q_raw, w.q_dtype, w.hq, self.cfg.scale, w.gqa_mapping,
                             w.indptr if indptr is None else indptr, w.indices if indices is None else indices,
                             w.last_page_len if lpl is None else lpl, seqs=seqs)


def header(run):
    """The CSR call's header in the workspace: chunk, wave items, overflow,
    slots, group items, group chunk, the nodes' wave items."""
    return [int(x) for x in run.ws[:28].view(dtype=__import__("torch").int32).cpu()]


def _check(run, got, ref, name):
    raw, err = max_abs_err(got, ref), excess_err(got, ref, run.w.q_dtype)
    print(f"[case] csr {name}: max abs err {raw:.3e}, beyond output rounding {err:.3e}", flush=True)
    assert np.all(np.isfinite(got)), "non-finite output"
    assert err <= TOL[run.w.q_dtype], f"{name}: {err}"


FORMATS = [(_lib.DTYPE_BF16, _lib.KV_BF16), (_lib.DTYPE_F16, _lib.KV_F16), (_lib.DTYPE_F32, _lib.KV_F32),
           (_lib.DTYPE_BF16, _lib.KV_FP8_E4M3), (_lib.DTYPE_BF16, _lib.KV_MXFP8),
           (_lib.DTYPE_F16, _lib.KV_FP8_E4M3)]


@pytest.mark.parametrize("shape", [(32, 4, 64), (32, 8, 128), (16, 2, 256), (32, 1, 64)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("fmt", FORMATS, ids=["bf16", "f16", "f32", "fp8", "mxfp8", "f16q-fp8"])
def test_random_trees(backend, shape, fmt):
    """Fork trees (shared pages appear in several tables) with partial last
    pages; (32, 1, 64) has 32 query heads per KV head, two row blocks per
    chunk."""
    hq, hkv, d = shape
    w = workloads.random_tree(31, hq, hkv, d, fmt[0], fmt[1], n_leaves=10, pool_pages=512)
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    _check(run, got, run.reference(), f"tree {shape} {fmt}")


@pytest.mark.parametrize("name", ["c1", "c2", "c3small", "c4small", "c5small"])
def test_configs(backend, name):
    w = {"c1": lambda: workloads.c1(),
         "c2": lambda: workloads.c2(),
         "c3small": lambda: workloads.c3(root_pages=40, levels=2, level_pages=3, pool_pages=4096),
         "c4small": lambda: workloads.c4(n_seqs=24, tmin=40, tmax=700, pool_pages=4096),
         "c5small": lambda: workloads.c5(requests=2, prefix_pages=40, beams=4, suffix_pages=5, pool_pages=2048)}[name]()
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    _check(run, got, run.reference(), name)


@pytest.mark.parametrize("case", ["many_short", "one_long", "mixed_64", "wide_lengths"])
def test_chunk_choice_shapes(backend, case):
    """Batches that reach the planning kernel's other branches: 1 500
    sequences (256 threads, page counts re-read past the ones kept in
    registers, several scan rounds), one 3 000-page sequence (the 64-states
    rule sets the chunk), 64 sequences with empty ones among them (one wave,
    full chunks written by the whole wave), 300 sequences of 1-700 pages
    (every last-chunk size).  Tables draw page ids with repeats, so pages
    are shared across sequences."""
    rng = np.random.default_rng({"many_short": 1, "one_long": 2, "mixed_64": 3, "wide_lengths": 4}[case])
    if case == "many_short":
        lens = rng.integers(1, 7, 1500)
    elif case == "one_long":
        lens = np.array([3000])
    elif case == "mixed_64":
        lens = rng.integers(0, 40, 64)
        lens[::7] = 0
    else:
        lens = rng.integers(1, 700, 300)
    pool_pages = int(max(64, lens.sum() // 2 + 8))
    tables = [rng.integers(0, pool_pages, int(n)).tolist() for n in lens]
    lpl = rng.integers(1, 17, len(lens)).astype(np.int32)
    w = workloads.custom(tables, 8, 2, 64, _lib.DTYPE_BF16, _lib.KV_BF16, pool_pages, last_page_len=lpl)
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    assert np.all(got[lens == 0] == 0)
    _check(run, got, run.reference(), case)


def test_c3_full(backend):
    """The headline tree from device tables, all 64 leaves against the
    oracle: the 512-page root is one group's shared pages (read once per KV
    head and 128-row block: 16 chunks x 8 heads x 2 blocks = 256 group
    items), each leaf's other 24 pages go to wave items."""
    w = workloads.c3()
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    h = header(run)
    print(f"[case] csr c3 header {h}", flush=True)
    # root: 256 group items of 32 pages; the 4 level-1 runs (64 rows, 8
    # pages) and 16 level-2 runs (16 rows): wave items of 16 rows, 4 x 8 x 4
    # + 16 x 8 x 1; each leaf's last 8 pages its own
    assert h[4] == 256 and h[5] == 32 and h[6] == 256
    _check(run, got, run.reference(), "c3 full")


def _grouped(run):
    """Items reading shared prefixes once: group items and nodes' wave items."""
    h = header(run)
    return h[4] + h[6]


def test_cascade_groups(backend):
    """Nodes of consecutive sequences: a common prefix of 8 pages or more
    makes one, 7 does not; a sequence that is its successor's prefix shares
    all but its last page; sequences that share a prefix but are not
    adjacent are read flat; duplicates share all but their last page; a node
    of 40 sequences x 8 heads of one KV head spans three 128-row blocks.
    Nodes of 16 rows are read by wave items, larger ones by group items."""
    import torch
    rng = np.random.default_rng(5)
    perm = iter(rng.permutation(4096).tolist())
    take = lambda n: [next(perm) for _ in range(n)]  # noqa: E731
    p20, p7, p30 = take(20), take(7), take(30)
    tables = []
    tables += [p20 + take(3) for _ in range(3)]             # group of 3, 20 shared pages
    tables += [p7 + take(2) for _ in range(2)]              # 7 shared: no group
    par = take(12)
    tables += [par, par + take(4)]                          # prefix: 11 shared pages
    x = take(9)
    tables += [x + take(2), take(5), x + take(3)]           # not adjacent: flat
    d = take(10)
    tables += [d, list(d)]                                  # duplicates: 9 shared
    tables += [p30 + take(1 + i % 3) for i in range(40)]    # 40 members
    lpl = rng.integers(1, 17, len(tables)).astype(np.int32)
    w = workloads.custom(tables, 8, 1, 64, _lib.DTYPE_BF16, _lib.KV_BF16, 4096, last_page_len=lpl)
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    h = header(run)
    print(f"[case] csr groups header {h}", flush=True)
    # group items, chunk 8 (items at most 256): 3 and 4 chunks of the 20- and
    # 30-page prefixes x 1 KV head x 1 and 3 row blocks; the 11- and 9-page
    # prefixes of two sequences (16 rows): one wave item each
    assert h[5] == 8 and h[4] == 3 * 1 + 4 * 3 and h[6] == 2
    _check(run, got, run.reference(), "groups")


@pytest.mark.parametrize("fmt", FORMATS, ids=["bf16", "f16", "f32", "fp8", "mxfp8", "f16q-fp8"])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_cascade_formats(backend, fmt, d):
    """A two-level tree (a root shared by every leaf, then pairs) in every
    format and head_dim: group items read the root; f32 queries have none
    (wave items only)."""
    rng = np.random.default_rng(d + fmt[1])
    perm = iter(rng.permutation(2048).tolist())
    take = lambda n: [next(perm) for _ in range(n)]  # noqa: E731
    root = take(37)
    tables = []
    for _ in range(6):
        mid = root + take(9)
        tables += [mid + take(1 + int(rng.integers(0, 4))) for _ in range(2)]
    lpl = rng.integers(1, 17, len(tables)).astype(np.int32)
    w = workloads.custom(tables, 16, 2, d, fmt[0], fmt[1], 2048, last_page_len=lpl)
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    assert (_grouped(run) > 0) == (fmt[0] != _lib.DTYPE_F32)
    _check(run, got, run.reference(), f"cascade d={d} {fmt}")


def test_bad_id_in_a_shared_prefix_zeros_the_group(backend):
    """A page id outside the pool inside a group's shared pages is in every
    member's table: all members get zeros and the status DH_EINVAL; a bad id
    in one member's own pages zeros that member only."""
    rng = np.random.default_rng(9)
    perm = iter(rng.permutation(1024).tolist())
    take = lambda n: [next(perm) for _ in range(n)]  # noqa: E731
    shared = take(16)
    tables = [shared + take(2) for _ in range(4)] + [take(5)]
    w = workloads.custom(tables, 8, 2, 64, _lib.DTYPE_BF16, _lib.KV_BF16, 1024)
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK and _grouped(run) > 0
    good = run.reference()
    _check(run, got, good, "shared ok")
    ix = w.indices.astype(np.int64).copy()
    for b in range(4):
        ix[w.indptr[b] + 5] = 5000                        # the same shared page in every member
    got, st = run.run(indices=ix)
    assert st == _lib.DH_EINVAL
    assert np.all(got[:4] == 0)
    _check(run, got[4:], good[4:], "bystander")
    ix = w.indices.astype(np.int64).copy()
    ix[w.indptr[2] + 16] = -3                             # member 2's own page
    got, st = run.run(indices=ix)
    assert st == _lib.DH_EINVAL
    assert np.all(got[2] == 0)
    keep = [0, 1, 3, 4]
    _check(run, got[keep], good[keep], "one member bad")


def test_empty_sequences_and_full_last_pages(backend):
    tables = [[], [3, 4, 5], [], [7], [6, 2]]
    w = workloads.custom(tables, 8, 2, 64, _lib.DTYPE_BF16, _lib.KV_BF16, 16, last_page_len=[1, 5, 16, 0, 9])
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    _check(run, got, run.reference(), "empty + lpl")
    # last_page_len NULL: every page full
    got, st = run.run(use_lpl=False)
    assert st == _lib.DH_OK
    _check(run, got, run.reference(lpl=np.full(5, 16, np.int32)), "lpl NULL")


def test_bad_ids_and_indptr_zero_their_sequences(backend):
    """A page id outside the pool (or negative) and a decreasing indptr make
    their sequences' outputs zero and the status DH_EINVAL; the other
    sequences are exact and nothing outside the pool is read."""
    tables = [[1, 2, 3], [4, 5], [6, 7, 8, 9], [10]]
    w = workloads.custom(tables, 8, 2, 64, _lib.DTYPE_BF16, _lib.KV_BF16, 16, last_page_len=[3, 7, 16, 2])
    run = CsrRun(w, backend)
    got, st = run.run()
    assert st == _lib.DH_OK
    good = run.reference()
    _check(run, got, good, "valid tables")
    for bad_id in (16, 1 << 30, -5):
        ix = w.indices.astype(np.int64).copy()
        ix[3] = bad_id                       # sequence 1's first page
        got, st = run.run(indices=ix)
        assert st == _lib.DH_EINVAL, bad_id
        assert np.all(got[1] == 0)
        keep = [0, 2, 3]
        _check(run, got[keep], good[keep], f"bad id {bad_id}")
    ip = w.indptr.astype(np.int64).copy()
    ip[2] = ip[1] - 1                        # sequence 1 ends before it starts
    got, st = run.run(indptr=ip)
    assert st == _lib.DH_EINVAL
    assert np.all(got[1] == 0)
    # the valid tables again: the status and outputs come back
    got, st = run.run()
    assert st == _lib.DH_OK
    _check(run, got, good, "valid again")


def test_tables_larger_than_the_workspace(backend):
    """A workspace sized for one page holds a handful of chunk slots (batch
    + 1, plus the cascade's allowance of one per sequence): tables that need
    more chunks of 256 pages leave every output zero with status DH_ENOMEM;
    a workspace below batch + 1 slots is refused on the host."""
    import torch
    tables = [list(range(1, 2400)), [2500]]
    w = workloads.custom(tables, 8, 2, 64, _lib.DTYPE_BF16, _lib.KV_BF16, 4096)
    run = CsrRun(w, backend, ws_pages=1)
    got, st = run.run()
    assert st == _lib.DH_ENOMEM
    assert np.all(got == 0)
    ix, ip, lp = run.tables()
    small = torch.empty(256, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(DhError) as e:
        decode_csr(backend, run.pool, run.cfg, run.q, ix, ip, lp, run.out, small)
    assert e.value.status == _lib.DH_EINVAL


def test_tables_change_between_calls(backend):
    """One workspace, tables that grow and shrink between calls: nothing of
    an earlier call's decomposition leaks into the next."""
    w = workloads.c2(branches=4, prefix_pages=60, suffix_pages=6, pool_pages=512)
    run = CsrRun(w, backend, ws_pages=2000)
    got, st = run.run()
    assert st == _lib.DH_OK
    _check(run, got, run.reference(), "c2 reduced")
    for cut in (1, 17, 45):
        keep = [b for b in range(w.batch)]
        tabs = [list(w.seq_pages(b))[:max(1, len(w.seq_pages(b)) - cut * (b + 1) % 50)] for b in keep]
        ip = np.concatenate([[0], np.cumsum([len(t) for t in tabs])]).astype(np.int64)
        ix = np.concatenate(tabs).astype(np.int64)
        lpl = np.array([(3 * b + cut) % 16 + 1 for b in keep], np.int32)
        got, st = run.run(indptr=ip, indices=ix, lpl=lpl)
        assert st == _lib.DH_OK
        _check(run, got, run.reference(indptr=ip.astype(np.uint32), indices=ix.astype(np.uint32), lpl=lpl),
               f"cut {cut}")
