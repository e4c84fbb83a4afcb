"""Error budget of the decode kernels' arithmetic at C5's shape (MXFP8 KV
with 1 % outliers at 20 sigma, bf16 queries, 64/8/128), CPU only.

A numpy emulation of what the kernels compute for one row: raw scores in
fp32, the lazy running max (moved only when a scaled score passes it by 32
log2 units for bf16 probabilities, 14 for f16), probabilities exp2(x - m)
rounded to the PV operand type, row sums and P.V accumulated in fp32, each
chunk's partial state stored as f16 scaled by 2^-k with its log2-sum-exp,
and the log-sum-exp merge in fp32; against the exact result in f64 from
the same dequantised K / V.  It pins which rounding carries the error:
bf16 probabilities (8 significant bits) dominate it, f16 probabilities
(11 bits, as the shared-prefix items of 8-bit pools use when V fits f16)
cut it by more than half, and the f16 partial states alone are smaller
still.  The dequantisation follows the oracle (E4M3 code x E8M0 scale,
oracle/oracle.c kv_elem); the kernels' own outputs are checked against the
oracle in test_gpu_properties.py (full-size C5) and test_gpu_decode.py.
"""
import numpy as np
import pytest

import oracle
from dendrite_amd import _lib, workloads

E4M3 = np.array([oracle.e4m3_to_float(c) for c in range(256)], np.float64)


def _bf16(x):
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def _kv(w, b):
    pages = w.seq_pages(b)
    data, sc = w.make_pages(pages)
    n, G = len(pages), w.d // 32
    codes = data.reshape(n, 2, w.hkv, 16, w.d)
    scale = np.ldexp(1.0, sc.reshape(n, 2, w.hkv, 16, G).astype(np.int64) - 127)
    vals = E4M3[codes] * np.repeat(scale, 32, axis=-1)
    vals = vals.transpose(1, 2, 0, 3, 4).reshape(2, w.hkv, n * 16, w.d)
    return vals[0], vals[1]


def _emulate(K, V, Q, chunks, f, rounding):
    """rounding(chunk index) -> (probability rounding, lazy slack)."""
    lses, states, exps = [], [], []
    for ci, (t0, t1) in enumerate(chunks):
        p_round, lazy = rounding(ci)
        m = thr = None
        L = np.zeros(len(Q), np.float32)
        O = np.zeros((len(Q), K.shape[1]), np.float32)
        for p0 in range(t0, t1, 32):
            p1 = min(p0 + 32, t1)
            r = (Q @ K[p0:p1].T).astype(np.float32)
            mx = r.max(axis=1)
            if m is None:
                m = (mx * f).astype(np.float32)
                thr = ((m + lazy) / f).astype(np.float32)
            else:
                mv = mx > thr
                mnew = (mx * f).astype(np.float32)
                alpha = np.exp2(m - mnew).astype(np.float32)
                L = np.where(mv, L * alpha, L)
                O = np.where(mv[:, None], O * alpha[:, None], O)
                m = np.where(mv, mnew, m)
                thr = np.where(mv, ((mnew + lazy) / f).astype(np.float32), thr)
            p = p_round(np.exp2((r.astype(np.float64) * f - m[:, None]).astype(np.float32)))
            L = (L + p.sum(axis=1, dtype=np.float32)).astype(np.float32)
            O = (O + (p.astype(np.float64) @ V[p0:p1]).astype(np.float32)).astype(np.float32)
        o = O / L[:, None]
        k = np.maximum(np.where(np.abs(o).max(axis=1) > 0, np.frexp(np.abs(o).max(axis=1))[1] - 15, 0), -100)
        states.append(_f16(o * np.ldexp(np.float32(1), -k)[:, None]))
        exps.append(k)
        lses.append((m + np.log2(L)).astype(np.float32))
    lses = np.stack(lses)
    wk = np.exp2(lses - lses.max(axis=0)).astype(np.float32)
    acc = sum((wk[s] * np.ldexp(np.float32(1), exps[s]))[:, None] * states[s] for s in range(len(chunks)))
    return acc / wk.sum(axis=0, dtype=np.float32)[:, None]


def _beyond_bf16_rounding(got, exact):
    half_ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(np.abs(exact), 1e-300))).astype(np.int64) - 8)
    return float((np.abs(_bf16(got).astype(np.float64) - exact) - half_ulp).max())


@pytest.fixture(scope="module")
def c5_rows():
    """Two beams of a C5 request (2 048-page prefix, as in the benchmark) and
    their exact outputs; chunks of 512 pages over the prefix, the suffix
    one chunk, as the planner cuts them."""
    w = workloads.c5(requests=1, beams=2)
    assert w.kv_format == _lib.KV_MXFP8 and w.q_dtype == _lib.DTYPE_BF16
    f = np.float32(1.4426950408889634 / np.sqrt(w.d))
    rows = []
    for b in range(w.batch):
        K, V = _kv(w, b)
        qb = (w.make_q()[b].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        T = (len(w.seq_pages(b)) - 1) * 16 + int(w.last_page_len[b] or 16)
        npre = 2048 * 16
        chunks = [(i, i + 8192) for i in range(0, npre, 8192)] + [(npre, T)]
        for h in range(w.hkv):
            Q = qb[[j for j in range(w.hq) if j % w.hkv == h]]
            s = (Q @ K[h][:T].T) / np.sqrt(w.d)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            exact = (p / p.sum(axis=1, keepdims=True)) @ V[h][:T]
            rows.append((K[h][:T], V[h][:T], Q, chunks, exact))
    return f, rows


def _max_err(c5_rows, rounding):
    f, rows = c5_rows
    return max(_beyond_bf16_rounding(_emulate(K, V, Q, ch, f, rounding), ex) for K, V, Q, ch, ex in rows)


def test_bf16_probabilities_dominate_the_error(c5_rows):
    bf16_all = _max_err(c5_rows, lambda ci: (_bf16, 32.0))
    f16_prefix = _max_err(c5_rows, lambda ci: (_bf16, 32.0) if ci == 4 else (_f16, 14.0))
    f32_p = _max_err(c5_rows, lambda ci: ((lambda p: np.asarray(p, np.float32)), 32.0))
    print(f"beyond bf16 output rounding: bf16 P {bf16_all:.3e}, f16 P in the prefix chunks {f16_prefix:.3e}, "
          f"fp32 P (f16 states only) {f32_p:.3e}")
    assert f16_prefix < 0.5 * bf16_all
    assert f32_p <= f16_prefix
    assert f16_prefix < 1.0e-2
