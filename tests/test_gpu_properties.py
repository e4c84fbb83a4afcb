"""Size-independent properties of the decode path at the benchmark sizes, the
maximum sequence length, and the largest configuration against the oracle:

- page placement: the same page contents stored at other pool slots (a
  permutation of page ids applied to the pool and the page lists) give
  bit-identical outputs, at the full C3 (bf16 tree) and C4 (FP8, 256
  sequences) sizes; the plan depends on the page lists only through which
  ids are equal, so a relabelling leaves the arithmetic unchanged;
- duplicated sequences (same page list, same query rows) give bit-identical
  output rows, shared prefix or not;
- a sequence of DH_MAX_SEQ_LEN tokens (8192 pages), alone and beside one that
  shares half of it, against the oracle;
- the full C5 configuration (MXFP8, 512 sequences, 32 prefixes of 2048 pages)
  against the oracle on sampled sequences.
Tolerance where the oracle is the reference: 2e-2 beyond bf16 output
rounding, as for every bf16 decode.
"""
import numpy as np
import pytest

from dendrite_amd import _lib, workloads
from tests._helpers import max_abs_err, TOL, GpuRun, excess_err

pytestmark = pytest.mark.gpu


def _relabelled(w, seed):
    """The workload with page ids permuted over the pool (same contents)."""
    perm = np.random.default_rng(seed).permutation(w.num_pool_pages).astype(np.uint32)
    ix = w.indices.copy()
    ok = ix != _lib.INVALID_PAGE
    ix[ok] = perm[ix[ok]]
    w2 = workloads.Workload(w.name + "-moved", w.hq, w.hkv, w.d, w.q_dtype, w.kv_format, w.num_pool_pages,
                            w.indptr.copy(), ix, w.last_page_len.copy(), w.seed, outlier=w.outlier,
                            outlier_every=w.outlier_every, gqa_mapping=w.gqa_mapping)
    return w2, perm


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_page_placement_does_not_change_outputs(backend, name):
    w = getattr(workloads, name)()
    print(f"[case] placement {name} batch={w.batch} pages={len(w.page_ids())}", flush=True)
    a = GpuRun(w, backend)
    out_a = a.run()
    w2, perm = _relabelled(w, 7)
    # the same page records, written at the permuted slots
    b = GpuRun(w2, backend, ids=perm[a.ids])
    b.pool.write_pages(perm[a.ids], a.data, a.scales)
    b.q = a.q
    out_b = b.run()
    assert np.array_equal(out_a.view(np.uint32), out_b.view(np.uint32))


@pytest.mark.parametrize("fmt", [_lib.KV_BF16, _lib.KV_FP8_E4M3], ids=["bf16", "fp8"])
def test_duplicated_sequences_give_identical_rows(backend, fmt):
    rng = np.random.default_rng(3)
    pages = rng.permutation(600)[:300].tolist()
    tables = [pages[:200], pages[:200], pages[:120] + pages[200:260], pages[:120] + pages[200:260], pages[260:]]
    w = workloads.custom(tables, 32, 8, 128, _lib.DTYPE_BF16, fmt, 600, last_page_len=[5, 5, 16, 16, 9])
    print(f"[case] duplicates fmt={fmt}", flush=True)
    run = GpuRun(w, backend)
    q = run.q_raw.copy()
    q[1] = q[0]
    q[3] = q[2]
    from tests._helpers import q_tensor
    run.q = q_tensor(q, w.q_dtype)
    run.q_raw = q
    out = run.run()
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    assert np.array_equal(out[2].view(np.uint32), out[3].view(np.uint32))
    assert excess_err(out, run.reference(), w.q_dtype) <= TOL[w.q_dtype]


def test_maximum_sequence_length(backend):
    n = _lib.MAX_SEQ_LEN // 16
    assert n == 8192
    rng = np.random.default_rng(4)
    pages = rng.permutation(n + 64).astype(np.uint32)
    tables = [pages[:n].tolist(), pages[:n // 2].tolist() + pages[n:n + 64].tolist()]
    w = workloads.custom(tables, 8, 2, 128, _lib.DTYPE_BF16, _lib.KV_BF16, n + 64, last_page_len=[16, 3])
    print(f"[case] max seq len {w.seq_len(0)} tokens", flush=True)
    assert w.seq_len(0) == _lib.MAX_SEQ_LEN
    run = GpuRun(w, backend)
    got = run.run()
    assert excess_err(got, run.reference(), w.q_dtype) <= TOL[w.q_dtype]


def test_c5_full_all_leaves(backend):
    """C5 at full size: all 512 leaves (32 requests x 16 beams) against the
    oracle."""
    w = workloads.c5()
    print(f"[case] c5 full batch={w.batch}", flush=True)
    run = GpuRun(w, backend)
    got = run.run()
    ref = run.reference()
    raw, err = max_abs_err(got, ref), excess_err(got, ref, w.q_dtype)
    print(f"[case] c5 full ({w.batch} leaves): max abs err {raw:.3e}, beyond output rounding {err:.3e}",
          flush=True)
    assert np.all(np.isfinite(got))
    assert err <= TOL[w.q_dtype]
