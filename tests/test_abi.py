"""The C ABI without a GPU: libdendrite_hip.so loads, exports every function
include/dendrite_hip.h declares, and its host-side entry points behave as
documented (no device compute is called here); likewise the test-data
library (libdendrite_testdata.so, include/dendrite_testdata.h), which the
backend library does not contain."""
import ctypes as C
import math
import os
import re

import numpy as np
import pytest
import torch

from dendrite_amd import _lib
from dendrite_amd.backend import AttentionConfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dendrite_hip.h")
TESTDATA_HEADER = os.path.join(ROOT, "include", "dendrite_testdata.h")


def _declared(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    names = set(re.findall(r"\b(dh_[a-z0-9_]+)\s*\(", text))
    typedefs = set(re.findall(r"typedef\s+(?:struct|enum)?\s*\w*\s*\{?[^;]*?\b(dh_[a-z0-9_]+)\s*;", text))
    return sorted(names - typedefs)


def test_library_exports_every_declared_function():
    L = _lib.lib()
    names = _declared()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and the ctypes signature table covers them all
    assert not [n for n in names if n not in _lib.SIGNATURES]


def test_testdata_library_is_separate():
    """The seeded generators are declared and exported by the test-data
    library only: the backend's header and library hold none of them."""
    T = _lib.testdata_lib()
    names = _declared(TESTDATA_HEADER)
    assert {"dh_synth_normal", "dh_synth_fill", "dh_synth_pages", "dh_testdata_last_error"} <= set(names)
    assert not [n for n in names if not hasattr(T, n)]
    assert not [n for n in names if n not in _lib.TESTDATA_SIGNATURES]
    assert not [n for n in _declared() if n.startswith("dh_synth")]
    assert not [n for n in ("dh_synth_normal", "dh_synth_fill", "dh_synth_pages") if hasattr(_lib.lib(), n)]
    assert T.dh_synth_pages(99, 1, 64, 0, None, 0, C.c_double(0.0), 0, None, None) == _lib.DH_EINVAL
    assert b"kv_format" in T.dh_testdata_last_error()


def test_version_and_errors():
    L = _lib.lib()
    assert b"gfx950" in C.string_at(L.dh_version())
    assert L.dh_attn_config_init(None, 8, 8, 64) == _lib.DH_EINVAL
    assert b"NULL" in C.string_at(L.dh_last_error())


@pytest.mark.parametrize("d", [64, 128, 256])
def test_config_scale_is_f32_inverse_sqrt(d):
    """backend.rs:37: scale = 1.0 / (head_dim as f32).sqrt(), in f32."""
    c = AttentionConfig(32, 8, d)
    assert c.scale == float(np.float32(1.0) / np.sqrt(np.float32(d)))
    assert c.num_queries_per_kv() == 4
    assert _lib.lib().dh_attn_config_num_queries_per_kv(C.byref(c.to_c())) == 4
    assert abs(c.scale - 1 / math.sqrt(d)) < 1e-7


def test_default_config():
    c = AttentionConfig.default()         # backend.rs:54-58
    assert (c.num_heads, c.num_kv_heads, c.head_dim) == (8, 8, 64)
    assert c.gqa_mapping == _lib.GQA_TILED


def test_no_device_is_reported_not_crashed():
    n = C.c_int(-1)
    assert _lib.lib().dh_device_count(C.byref(n)) == _lib.DH_OK
    if n.value > 0:
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    assert _lib.lib().dh_create(0, C.byref(h)) == _lib.DH_EUNSUPPORTED
    assert not h.value
    assert _lib.lib().dh_is_available() == 0


def test_synth_normal_is_deterministic_and_normal():
    L = _lib.testdata_lib()
    a = np.array([L.dh_synth_normal(7, i) for i in range(20000)])
    assert np.array_equal(a, [L.dh_synth_normal(7, i) for i in range(20000)])
    assert abs(a.mean()) < 0.03 and abs(a.std() - 1) < 0.03
    out = np.zeros(20000, dtype=np.uint16)
    assert L.dh_synth_fill(out.ctypes.data, _lib.DTYPE_BF16, 7, 0, 20000) == 0
    want = torch.from_numpy(a).float().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("fmt", [_lib.KV_FP8_E4M3, _lib.KV_MXFP8])
def test_synth_fp8_pages_round_like_torch(fmt):
    """The synthetic page encoder rounds to nearest even and saturates at 448,
    like torch's float8_e4m3fn conversion of the pre-clamped value."""
    L = _lib.testdata_lib()
    hkv, d = 2, 64
    ids = np.array([3, 9], dtype=np.uint32)
    page_elems = 2 * hkv * 16 * d
    data = np.zeros((2, page_elems), dtype=np.uint8)
    sbytes = 2 * hkv * 4 if fmt == _lib.KV_FP8_E4M3 else 2 * hkv * 16 * (d // 32)
    scales = np.zeros((2, sbytes), dtype=np.uint8)
    assert L.dh_synth_pages(fmt, hkv, d, 5, ids.ctypes.data_as(_lib._PU32), 2, C.c_double(20.0), 50, data.ctypes.data,
                            scales.ctypes.data) == 0
    for row, pid in enumerate(ids):
        x = np.array([L.dh_synth_normal(5, int(pid) * page_elems + e) for e in range(page_elems)],
                     dtype=np.float32)
        x = x.reshape(2 * hkv, 16 * d)
        codes = data[row].reshape(2 * hkv, 16 * d)
        if fmt == _lib.KV_FP8_E4M3:
            sc = scales[row].view(np.float32)
            # outliers are placed by a hash; recover them from the codes' magnitudes
            for blk in range(2 * hkv):
                xs = torch.from_numpy(x[blk]).double()
                dec = torch.from_numpy(codes[blk]).view(torch.float8_e4m3fn).double() * float(sc[blk])
                ok = (dec.abs() < 19.0) & (xs.abs() < 19.0)
                want = (xs / float(sc[blk])).clamp(-448, 448).float().to(torch.float8_e4m3fn)
                got = torch.from_numpy(codes[blk]).view(torch.float8_e4m3fn)
                assert torch.equal(got.view(torch.uint8)[ok], want.view(torch.uint8)[ok])
        else:
            e = scales[row].reshape(2 * hkv, 16 * d // 32).astype(np.float64) - 127
            sc = np.repeat(np.ldexp(1.0, e.astype(np.int64)), 32, axis=1)
            got = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn)
            dec = got.double().numpy() * sc
            ok = torch.from_numpy((np.abs(dec) < 19.0) & (np.abs(x) < 19.0))
            # OCP MX: elements beyond the E4M3 range after scaling saturate
            want = torch.from_numpy(x / sc).clamp(-448, 448).float().to(torch.float8_e4m3fn)
            assert torch.equal(got.view(torch.uint8)[ok], want.view(torch.uint8)[ok])
            # scale = 2^(floor(log2 amax) - 8) of each group of 32 (checked on
            # groups without outliers)
            amax = np.abs(x).reshape(2 * hkv, -1, 32).max(axis=2)
            clean = ok.numpy().reshape(2 * hkv, -1, 32).all(axis=2)
            assert np.array_equal(e[clean], (np.floor(np.log2(amax)) - 8)[clean])


def test_tree_entry_points_take_16_token_blocks_only():
    """Decode pages hold 16 tokens: the tree entry points refuse trees of
    other block sizes (an 8-token tree's last_page_len would be wrong for a
    16-token page) with DH_EUNSUPPORTED, before touching any device."""
    from dendrite_amd.cache import KvCache, KvCacheConfig, TreeState
    L = _lib.lib()
    for tpb, want in ((8, _lib.DH_EUNSUPPORTED), (16, _lib.DH_OK)):
        cache = KvCache(KvCacheConfig(num_layers=1, num_kv_heads=1, head_dim=64, max_blocks=16,
                                      tokens_per_block=tpb))
        tree = TreeState(cache, tpb)
        assert tree.tokens_per_block == tpb
        leaf = tree.fork(0).node_id
        for t in range(12):
            tree.append_token(leaf, t)
        nodes = np.array([leaf], dtype=np.uint64)
        lpl = np.zeros(1, dtype=np.int32)
        rc = L.dh_tree_last_page_len(tree._h, nodes.ctypes.data_as(_lib._PU64), 1,
                                     lpl.ctypes.data_as(C.POINTER(C.c_int32)))
        assert rc == want
        if rc == _lib.DH_OK:
            assert lpl[0] == 12
        cfg = AttentionConfig(8, 8, 64).to_c()
        plan = C.c_void_p()
        rc = L.dh_plan_create_tree(None, C.byref(cfg), None, tree._h, nodes.ctypes.data_as(_lib._PU64), 1, 1,
                                   None, C.byref(plan))
        if tpb != 16:
            assert rc == _lib.DH_EUNSUPPORTED and b"16" in C.string_at(L.dh_last_error())
        assert not plan.value


def test_csr_workspace_size_grows_then_caps():
    """dh_csr_workspace_size (host-only): 0 for an empty batch; grows with
    the batch and with the tables' page count until the slot cap; a workspace
    for many pages serves fewer."""
    from dendrite_amd.backend import AttentionConfig, csr_workspace_size
    cfg = AttentionConfig(32, 8, 128)
    assert csr_workspace_size(cfg, 0, 100) == 0
    sizes = [csr_workspace_size(cfg, 64, t) for t in (1, 8, 64, 512, 4096, 34304, 1 << 20, 1 << 24)]
    assert all(s > 0 and s % 256 == 0 for s in sizes)
    assert sizes == sorted(sizes)
    assert sizes[-1] == sizes[-2] or sizes[-1] - sizes[-2] < sizes[-2]   # capped slot counts
    assert csr_workspace_size(cfg, 65, 34304) > sizes[5]
    # f32 queries keep fp32 partial states: larger (one sequence: no cascade
    # room for either)
    cfg32 = AttentionConfig(32, 8, 128)
    cfg32.q_dtype = _lib.DTYPE_F32
    cfg32.kv_format = _lib.KV_F32
    assert csr_workspace_size(cfg32, 1, 34304) > csr_workspace_size(cfg, 1, 34304)
    # 16-bit queries over 2..512 sequences may find shared prefixes: room for
    # their chunks (f32 queries never group, so their larger states do not
    # make up for it here)
    assert csr_workspace_size(cfg, 64, 34304) > csr_workspace_size(cfg32, 64, 34304)
    assert csr_workspace_size(cfg, 513, 34304) < csr_workspace_size(cfg, 512, 34304)
