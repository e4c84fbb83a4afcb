"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

How each oracle function is pinned:
  oracle_e4m3   all 256 codes against torch.float8_e4m3fn (tests/golden/
                fp8_tables.npz); the OCP range facts of quantization/fp8.rs:39-52
  oracle_e8m0   all 256 codes against torch.float8_e8m0fnu (same fixture)
  oracle_bf16,  all 65536 bit patterns against torch's bfloat16 / float16
  oracle_f16
  oracle_decode the golden decode cases (torch CPU scaled_dot_product_attention
                in f64 on the gathered, dequantised K/V: tests/golden/
                decode_cases.npz), plus known answers a plausible mistake
                fails: one-hot logits select one token's V row exactly (a
                wrong page, slot, plane or head index changes the integers
                read back), all-equal keys give the mean of V, an empty or
                all-INVALID table gives zeros, a token beyond last_page_len
                never contributes, both GQA mappings
  oracle_decode_candle  the same golden cases at f32 tolerance
  oracle_merge  against attention over the concatenation of the two halves
                (closed form of cascade.rs:116-124), identity of an empty
                (-inf) side, commutativity, and the reference formula's NaN
                for two empty sides (the product special-cases that)
Everything here runs on the CPU.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
INVALID = oracle.INVALID


def _golden_cases():
    z = np.load(os.path.join(GOLDEN, "decode_cases.npz"))
    names = sorted({k.split("/")[0] for k in z.files})
    return {n: {k.split("/")[1]: z[k] for k in z.files if k.startswith(n + "/")} for n in names}


CASES = _golden_cases()


def _run_case(c, mode="f64"):
    hq, hkv, d, q_dtype, fmt, gqa, pool_pages = (int(x) for x in c["meta"])
    scales = c["scales"] if c["scales"].shape[1] else None
    pv = oracle.PoolView(c["ids"], c["data"], scales, pool_pages, fmt, hkv, d)
    return oracle.decode(pv, c["q"], q_dtype, hq, float(c["scale"][0]), gqa, c["indptr"],
                         c["indices"], c["last_page_len"], mode=mode)


# ----------------------------------------------------------------- codecs
def test_e4m3_all_codes_match_torch():
    want = np.load(os.path.join(GOLDEN, "fp8_tables.npz"))["e4m3"]
    got = np.array([oracle.e4m3_to_float(c) for c in range(256)])
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert set(np.flatnonzero(nan)) == {0x7F, 0xFF}
    assert np.array_equal(got[~nan], want[~nan].astype(np.float64))
    # quantization/fp8.rs:39-52: max 448, smallest subnormal 2^-9
    assert np.nanmax(got) == 448.0 and got[1] == 2.0 ** -9


def test_e8m0_all_codes_match_torch():
    want = np.load(os.path.join(GOLDEN, "fp8_tables.npz"))["e8m0"]
    got = np.array([oracle.e8m0_to_float(c) for c in range(256)])
    assert np.isnan(got[255]) and np.isnan(want[255])
    assert np.array_equal(got[:255], want[:255].astype(np.float64))


def test_bf16_and_f16_all_patterns_match_torch():
    pats = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    L = oracle.lib()
    for fn, dt in ((L.oracle_bf16, torch.bfloat16), (L.oracle_f16, torch.float16)):
        want = pats.view(dt).double().numpy()
        got = np.array([fn(i) for i in range(65536)])
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan], want[~nan])


# ------------------------------------------------------------ golden cases
@pytest.mark.parametrize("name", sorted(CASES))
def test_decode_matches_golden(name):
    c = CASES[name]
    got = _run_case(c)
    assert got.shape == c["out"].shape
    np.testing.assert_allclose(got, c["out"], rtol=0, atol=1e-10)


@pytest.mark.parametrize("name", sorted(CASES))
def test_decode_candle_order_matches_golden(name):
    c = CASES[name]
    for mode in ("candle", "stream"):
        got = _run_case(c, mode=mode)
        np.testing.assert_allclose(got, c["out"], rtol=0, atol=1e-4)


def test_golden_single_token_is_its_v_row():
    c = CASES["f32_one_token"]
    hq, hkv, d = (int(x) for x in c["meta"][:3])
    page = c["data"][0].view(np.float32).reshape(2, hkv, 16, d)
    for h in range(hq):
        assert np.array_equal(c["out"][0, h], page[1, h % hkv, 0].astype(np.float64))


def test_golden_empty_table_is_zero():
    c = CASES["bf16_tree"]
    assert not np.any(c["out"][3])


# ---------------------------------------------------------- known answers
def _f32_pool(pages: dict, hkv: int, d: int, pool_pages: int):
    ids = sorted(pages)
    data = np.stack([pages[i].astype(np.float32).reshape(-1).view(np.uint8) for i in ids])
    return oracle.PoolView(np.array(ids, dtype=np.uint32), data, None, pool_pages, oracle.F32, hkv, d)


def _one_hot_case(gqa):
    """V rows encode (page, slot, head) as exact small integers; for query head
    h and target token t only K[t] aligns with q, with a logit margin of 100."""
    hq, hkv, d = 8, 2, 32
    rng = np.random.Generator(np.random.PCG64(5))
    ids = [int(x) for x in rng.permutation(40)[:6]]
    pages = {}
    for pid in ids:
        p = np.zeros((2, hkv, 16, d))
        for h in range(hkv):
            for s in range(16):
                p[0, h, s, :] = 0.0
                p[1, h, s, :] = pid * 1000 + s * 10 + h + np.arange(d) * 1e5
        pages[pid] = p
    table = ids[:4]
    lpl = 9
    # target token of query head h: page table[h % 4], slot (3 h + 1) % 16
    # (on the last page kept below last_page_len)
    q = np.zeros((1, hq, d), dtype=np.float32)
    want = np.zeros((hq, d))
    for h in range(hq):
        kh = h % hkv if gqa == 0 else h // (hq // hkv)
        j = h % 4
        slot = (3 * h + 1) % 16 if j < 3 else (3 * h + 1) % lpl
        pages[table[j]][0, kh, slot, h] = 1.0
        q[0, h, h] = 1000.0                       # logit 1000 * scale(~0.177) = 177
        want[h] = pages[table[j]][1, kh, slot]
    # a token beyond last_page_len with a larger logit must not contribute
    for h in range(hq):
        kh = h % hkv if gqa == 0 else h // (hq // hkv)
        pages[table[3]][0, kh, 15, h] = 5.0
    pv = _f32_pool(pages, hkv, d, 64)
    indptr = np.array([0, 4], dtype=np.uint32)
    return pv, q, hq, gqa, indptr, np.array(table, dtype=np.uint32), np.array([lpl], dtype=np.int32), want


@pytest.mark.parametrize("gqa", [0, 1], ids=["tiled", "interleaved"])
def test_one_hot_selects_exact_v_row(gqa):
    pv, q, hq, gqa, indptr, indices, lpl, want = _one_hot_case(gqa)
    scale = float(np.float32(1 / math.sqrt(32)))
    got = oracle.decode(pv, q, oracle.F32, hq, scale, gqa, indptr, indices, lpl)
    np.testing.assert_array_equal(got[0].astype(np.float32), want.astype(np.float32))
    got32 = oracle.decode(pv, q, oracle.F32, hq, scale, gqa, indptr, indices, lpl, mode="candle")
    np.testing.assert_array_equal(got32[0], want.astype(np.float32))


def test_gqa_mappings_differ():
    """The two mappings must give different results on the same input (so a
    swapped mapping cannot pass either test)."""
    pv, q, hq, _, indptr, indices, lpl, _ = _one_hot_case(0)
    a = oracle.decode(pv, q, oracle.F32, hq, 0.17677669, 0, indptr, indices, lpl)
    b = oracle.decode(pv, q, oracle.F32, hq, 0.17677669, 1, indptr, indices, lpl)
    assert not np.array_equal(a, b)


def test_all_equal_keys_give_mean_of_v():
    hkv, d, hq = 2, 64, 4
    rng = np.random.Generator(np.random.PCG64(9))
    pages = {}
    k = rng.standard_normal(d)
    for pid in (3, 17, 8):
        p = np.empty((2, hkv, 16, d))
        p[0] = k
        p[1] = rng.integers(-8, 8, size=(hkv, 16, d))
        pages[pid] = p
    pv = _f32_pool(pages, hkv, d, 32)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    indices = np.array([17, 3, 8], dtype=np.uint32)
    got = oracle.decode(pv, q, oracle.F32, hq, 0.125, 0, np.array([0, 3], dtype=np.uint32), indices,
                        np.array([5], dtype=np.int32))
    for h in range(hq):
        rows = [pages[17][1, h % hkv], pages[3][1, h % hkv], pages[8][1, h % hkv, :5]]
        np.testing.assert_allclose(got[0, h], np.concatenate(rows).mean(axis=0), atol=1e-12)


def test_empty_and_all_invalid_tables_give_zeros():
    pages = {1: np.ones((2, 1, 16, 32))}
    pv = _f32_pool(pages, 1, 32, 8)
    q = np.ones((2, 2, 32), dtype=np.float32)
    indptr = np.array([0, 0, 2], dtype=np.uint32)
    indices = np.array([INVALID, INVALID], dtype=np.uint32)
    got = oracle.decode(pv, q, oracle.F32, 2, 0.5, 0, indptr, indices, np.array([16, 16], dtype=np.int32))
    assert not np.any(got)


def test_invalid_id_is_skipped():
    """An INVALID entry contributes nothing; the rest of the table is read in
    order (backend.rs:228-233)."""
    rng = np.random.Generator(np.random.PCG64(4))
    pages = {i: rng.standard_normal((2, 1, 16, 32)) for i in (2, 5)}
    pv = _f32_pool(pages, 1, 32, 8)
    q = rng.standard_normal((1, 2, 32)).astype(np.float32)
    lpl = np.array([7], dtype=np.int32)
    a = oracle.decode(pv, q, oracle.F32, 2, 0.5, 0, np.array([0, 3], dtype=np.uint32),
                      np.array([2, INVALID, 5], dtype=np.uint32), lpl)
    b = oracle.decode(pv, q, oracle.F32, 2, 0.5, 0, np.array([0, 2], dtype=np.uint32),
                      np.array([2, 5], dtype=np.uint32), lpl)
    np.testing.assert_array_equal(a, b)


def test_absent_page_is_reported():
    pv = _f32_pool({1: np.zeros((2, 1, 16, 32))}, 1, 32, 8)
    with pytest.raises(ValueError):
        oracle.decode(pv, np.zeros((1, 1, 32), np.float32), oracle.F32, 1, 0.5, 0,
                      np.array([0, 1], dtype=np.uint32), np.array([3], dtype=np.uint32), None)


# ------------------------------------------------------------------- merge
def _attend(q, K, V, scale):
    s = K @ q * scale
    m = s.max()
    w = np.exp(s - m)
    return (w @ V) / w.sum(), m + math.log(w.sum())


def test_merge_equals_attention_over_concatenation():
    rng = np.random.Generator(np.random.PCG64(3))
    d, scale = 16, 0.25
    for split in (1, 7, 19):
        K = rng.standard_normal((20, d))
        V = rng.standard_normal((20, d))
        q = rng.standard_normal(d)
        o_all, lse_all = _attend(q, K, V, scale)
        o1, l1 = _attend(q, K[:split], V[:split], scale)
        o2, l2 = _attend(q, K[split:], V[split:], scale)
        for k in range(d):
            o, lse = oracle.merge(o1[k], l1, o2[k], l2)
            assert abs(o - o_all[k]) < 1e-5
            assert abs(lse - lse_all) < 1e-5


def test_merge_identity_and_commutativity():
    ninf = float("-inf")
    o, lse = oracle.merge(0.75, 2.5, 123.0, ninf)
    assert o == np.float32(0.75) and lse == np.float32(2.5)
    a = oracle.merge(0.3, 1.0, -2.0, 3.0)
    b = oracle.merge(-2.0, 3.0, 0.3, 1.0)
    assert a == b


def test_merge_of_two_empty_sides_is_nan_in_the_reference_formula():
    """cascade.rs:116-124 evaluates exp(-inf - -inf); the product's merge must
    special-case it (an empty segment pair stays empty: o = 0, lse = -inf)."""
    o, lse = oracle.merge(0.0, float("-inf"), 0.0, float("-inf"))
    assert math.isnan(o) and math.isnan(lse)
