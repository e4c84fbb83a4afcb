"""TEST INFRASTRUCTURE ONLY: the CPU oracle of the paged decode path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The product
package dendrite_amd never imports it.

oracle.c restates ReferenceBackend::decode (crates/dendrite-core/src/attention/
backend.rs:206-283) in f64 (parity) and in candle's f32 op order (baseline);
block_model.py restates the block pool / block table / tree semantics.  How
each function is pinned (golden vectors, known answers, library routines,
closed forms) is listed in the header of tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
SOURCE = os.path.join(HERE, "oracle.c")

F16, BF16, F32, FP8, MX = 0, 1, 2, 3, 4
INVALID = 0xFFFFFFFF


def build() -> str:
    """Compile oracle.c with gcc (OpenMP) into oracle/liboracle.so."""
    tmp = LIB_PATH + ".tmp"
    subprocess.run(["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-Wall", SOURCE, "-o", tmp, "-lm"],
                   check=True, capture_output=True, text=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.oracle_e4m3.restype = C.c_double
        L.oracle_e4m3.argtypes = [C.c_uint8]
        L.oracle_e8m0.restype = C.c_double
        L.oracle_e8m0.argtypes = [C.c_uint8]
        L.oracle_bf16.restype = C.c_double
        L.oracle_bf16.argtypes = [C.c_uint16]
        L.oracle_f16.restype = C.c_double
        L.oracle_f16.argtypes = [C.c_uint16]
        common = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                  C.c_void_p, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32, C.c_void_p, C.c_void_p,
                  C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]
        L.oracle_decode.restype = C.c_int
        L.oracle_decode.argtypes = common + [C.c_void_p, C.c_int]
        L.oracle_decode_candle.restype = C.c_int
        L.oracle_decode_candle.argtypes = common + [C.c_void_p, C.c_int, C.c_int]
        L.oracle_merge.restype = None
        L.oracle_merge.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float,
                                   C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.oracle_num_threads.restype = C.c_int
        L.oracle_e4m3_encode.restype = C.c_uint8
        L.oracle_e4m3_encode.argtypes = [C.c_float]
        L.oracle_write_pages.restype = C.c_int
        L.oracle_write_pages.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32,
                                         C.c_void_p, C.c_void_p]
        _lib = L
    return _lib


def e4m3_to_float(code: int) -> float:
    return lib().oracle_e4m3(code)


def e8m0_to_float(code: int) -> float:
    return lib().oracle_e8m0(code)


def merge(o1: float, lse1: float, o2: float, lse2: float) -> tuple[float, float]:
    o, lse = C.c_float(), C.c_float()
    lib().oracle_merge(o1, lse1, o2, lse2, C.byref(o), C.byref(lse))
    return o.value, lse.value


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class PoolView:
    """Host copy of the referenced pages: data/scales rows plus id -> row map."""

    def __init__(self, page_ids, data, scales, num_pool_pages, fmt, hkv, d):
        self.page_ids = np.ascontiguousarray(page_ids, dtype=np.uint32)
        self.data = np.ascontiguousarray(data)
        self.scales = None if scales is None else np.ascontiguousarray(scales)
        self.fmt, self.hkv, self.d = fmt, hkv, d
        self.num_pool_pages = num_pool_pages
        self.page_map = np.full(num_pool_pages, INVALID, dtype=np.uint32)
        self.page_map[self.page_ids] = np.arange(len(self.page_ids), dtype=np.uint32)


def decode(pool: PoolView, q, q_dtype, hq, scale, gqa, indptr, indices, last_page_len=None,
           seqs=None, threads=None, mode="f64"):
    """Runs the oracle over sequences `seqs` (default all).  Returns float64
    (mode "f64") or float32 (modes "candle", "stream") array [n][hq][d]."""
    L = lib()
    indptr = np.ascontiguousarray(indptr, dtype=np.uint32)
    indices = np.ascontiguousarray(indices, dtype=np.uint32)
    lpl = None if last_page_len is None else np.ascontiguousarray(last_page_len, dtype=np.int32)
    batch = len(indptr) - 1
    sq = None if seqs is None else np.ascontiguousarray(seqs, dtype=np.uint32)
    n = batch if sq is None else len(sq)
    q = np.ascontiguousarray(q)
    threads = threads or L.oracle_num_threads()
    args = [_ptr(pool.data), _ptr(pool.scales), _ptr(pool.page_map), pool.num_pool_pages, pool.fmt,
            pool.hkv, pool.d, _ptr(q), q_dtype, hq, float(scale), gqa, _ptr(indptr), _ptr(indices),
            _ptr(lpl), batch, _ptr(sq), n]
    if mode == "f64":
        out = np.zeros((n, hq, pool.d), dtype=np.float64)
        rc = L.oracle_decode(*args, _ptr(out), threads)
    else:
        out = np.zeros((n, hq, pool.d), dtype=np.float32)
        rc = L.oracle_decode_candle(*args, _ptr(out), threads, 1 if mode == "candle" else 0)
    if rc != 0:
        raise ValueError("oracle: a referenced page is absent from the pool view")
    return out


def e4m3_encode(x: float) -> int:
    """E4M3 code of a float: nearest finite value, ties to even, saturating."""
    return lib().oracle_e4m3_encode(x)


def scale_record_bytes(fmt: int, hkv: int, d: int) -> int:
    return {FP8: 2 * hkv * 4, MX: 2 * hkv * 16 * (d // 32)}.get(fmt, 0)


def write_pages(fmt: int, hkv: int, d: int, src: np.ndarray):
    """The page write rule on float pages src [n][2][hkv][16][d]: returns
    (data uint8 [n, page_bytes], scales uint8 [n, scale_bytes] or None)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    n = src.shape[0]
    eb = {F32: 4, BF16: 2, F16: 2, FP8: 1, MX: 1}[fmt]
    data = np.zeros((n, 2 * hkv * 16 * d * eb), dtype=np.uint8)
    sb = scale_record_bytes(fmt, hkv, d)
    scales = np.zeros((n, max(sb, 1)), dtype=np.uint8)
    rc = lib().oracle_write_pages(fmt, hkv, d, src.ctypes.data, n, data.ctypes.data, scales.ctypes.data)
    assert rc == 0, "bad format"
    return data, (scales if sb else None)
