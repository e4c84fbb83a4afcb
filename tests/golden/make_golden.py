"""Writes the golden fixtures under tests/golden/ from library routines only.

    python tests/golden/make_golden.py

The reference path (ReferenceBackend::decode on candle, crates/dendrite-core/
src/attention/backend.rs:206-283) is Rust and cannot run here, and its own
tests hold no numeric vectors for it, so the expected outputs are computed with
torch's CPU scaled_dot_product_attention in float64 on the dequantised,
gathered K/V; nothing from this repository's oracle or product is used.

fp8_tables.npz
  e4m3[256]   float32 value of every E4M3 (OCP FN) code, via torch.float8_e4m3fn
  e8m0[256]   float32 value of every E8M0 scale code, via torch.float8_e8m0fnu
decode_cases.npz  (keys "<case>/<field>")
  meta     int64 [hq, hkv, d, q_dtype, kv_format, gqa, num_pool_pages]
  scale    float64 [1]: f32(1/sqrt(d)) applied in f64, as backend.rs:37, :214
  ids      uint32 [n]: pool ids present; data uint8 [n][page_bytes] in the
           pool layout [K|V][kv_head][16][d]; scales uint8 [n][scale_bytes]
           (FP8: f32 per (plane, head); MXFP8: E8M0 per 32 along d)
  indptr, indices (uint32, CSR block tables, INVALID = 0xFFFFFFFF skipped),
  last_page_len (int32, valid tokens of each table's last page)
  q        raw bytes of q [B][hq][d] in q_dtype
  out      float64 [B][hq][d]: the expected output
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
INVALID = 0xFFFFFFFF
F16, BF16, F32, FP8, MX = 0, 1, 2, 3, 4          # q dtype / kv format codes of the C ABI
TILED, INTERLEAVED = 0, 1


def tables() -> None:
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    e4m3 = codes.view(torch.float8_e4m3fn).float().numpy()
    e8m0 = codes.view(torch.float8_e8m0fnu).float().numpy()
    np.savez_compressed(os.path.join(HERE, "fp8_tables.npz"), e4m3=e4m3, e8m0=e8m0)


def _encode_pages(rng, fmt, n, hkv, d, outlier_every=0):
    """Returns (raw bytes [n][page_bytes], scale bytes or None, dequantised f64 [n][2][hkv][16][d])."""
    x = torch.from_numpy(rng.standard_normal((n, 2, hkv, 16, d)))
    if outlier_every:
        mask = torch.from_numpy(rng.integers(0, outlier_every, size=x.shape) == 0)
        x = torch.where(mask, torch.sign(x) * 20.0, x)
    if fmt == F32:
        t = x.float()
        return t.view(torch.uint8).reshape(n, -1).numpy(), None, t.double()
    if fmt in (BF16, F16):
        t = x.to(torch.bfloat16 if fmt == BF16 else torch.float16)
        return t.view(torch.uint8).reshape(n, -1).numpy(), None, t.double()
    if fmt == FP8:
        amax = x.abs().amax(dim=(3, 4), keepdim=True)
        sc = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax)).float()
        e = (x / sc.double()).clamp(-448, 448).to(torch.float8_e4m3fn)
        deq = e.double() * sc.double()
        return (e.view(torch.uint8).reshape(n, -1).numpy(),
                sc.reshape(n, 2 * hkv).view(torch.uint8).reshape(n, -1).numpy(), deq)
    # MXFP8: E8M0 scale per 32 consecutive elements along d, 2^(floor(log2 amax) - 8)
    g = x.reshape(n, 2, hkv, 16, d // 32, 32)
    amax = g.abs().amax(dim=-1, keepdim=True)
    ex = torch.where(amax > 0, torch.floor(torch.log2(amax)) - 8, torch.full_like(amax, -127.0))
    ex = ex.clamp(-127, 127)
    e = (g / torch.pow(2.0, ex)).clamp(-448, 448).to(torch.float8_e4m3fn)
    deq = (e.double() * torch.pow(2.0, ex)).reshape(n, 2, hkv, 16, d)
    scales = (ex + 127).to(torch.uint8).reshape(n, -1).numpy()
    return e.view(torch.uint8).reshape(n, -1).numpy(), scales, deq


def _expected(deq_by_id, q, hq, hkv, d, scale, gqa, indptr, indices, lpl):
    B = len(indptr) - 1
    out = np.zeros((B, hq, d))
    r = hq // hkv
    for b in range(B):
        ids = indices[indptr[b]:indptr[b + 1]]
        ks, vs = [], []
        for j, pid in enumerate(ids):
            if pid == INVALID:
                continue
            nt = int(lpl[b]) if j == len(ids) - 1 else 16
            nt = 16 if nt == 0 else nt
            page = deq_by_id[int(pid)]
            ks.append(page[0, :, :nt])
            vs.append(page[1, :, :nt])
        if not ks:
            continue                                   # empty -> zeros (backend.rs:218-222)
        K = torch.cat(ks, dim=1)                        # [hkv][T][d]
        V = torch.cat(vs, dim=1)
        if gqa == TILED:
            K, V = K.repeat(r, 1, 1), V.repeat(r, 1, 1)     # head h uses kv head h % hkv
        else:
            K, V = K.repeat_interleave(r, 0), V.repeat_interleave(r, 0)   # h // r
        qq = torch.from_numpy(q[b]).unsqueeze(1)        # [hq][1][d]
        o = torch.nn.functional.scaled_dot_product_attention(qq, K, V, scale=scale)
        out[b] = o[:, 0].numpy()
    return out


def _q(rng, B, hq, d, q_dtype):
    x = torch.from_numpy(rng.standard_normal((B, hq, d)))
    t = x.to({F32: torch.float32, BF16: torch.bfloat16, F16: torch.float16}[q_dtype])
    return t.view(torch.uint8).numpy().reshape(B, -1), t.double().numpy()


def case(store, name, seed, hq, hkv, d, q_dtype, fmt, gqa, pool_pages, tables_, lpl, outlier_every=0):
    rng = np.random.Generator(np.random.PCG64(seed))
    ids = sorted({p for t in tables_ for p in t if p != INVALID})
    data, scales, deq = _encode_pages(rng, fmt, len(ids), hkv, d, outlier_every)
    deq_by_id = {pid: deq[i] for i, pid in enumerate(ids)}
    indptr = np.zeros(len(tables_) + 1, dtype=np.uint32)
    for i, t in enumerate(tables_):
        indptr[i + 1] = indptr[i] + len(t)
    indices = np.array([p for t in tables_ for p in t], dtype=np.uint32)
    lpl = np.asarray(lpl, dtype=np.int32)
    q_raw, q64 = _q(rng, len(tables_), hq, d, q_dtype)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    out = _expected(deq_by_id, q64, hq, hkv, d, scale, gqa, indptr, indices, lpl)
    f = {"meta": np.array([hq, hkv, d, q_dtype, fmt, gqa, pool_pages], dtype=np.int64),
         "scale": np.array([scale]), "ids": np.array(ids, dtype=np.uint32), "data": data,
         "scales": scales if scales is not None else np.zeros((len(ids), 0), dtype=np.uint8),
         "indptr": indptr, "indices": indices, "last_page_len": lpl, "q": q_raw, "out": out}
    for k, v in f.items():
        store[f"{name}/{k}"] = v


def decode_cases() -> None:
    s = {}
    rng = np.random.Generator(np.random.PCG64(2024))
    perm = [int(p) for p in rng.permutation(64)]
    # 1. one f32 sequence over 5 shuffled pages
    case(s, "f32_single", 1, 8, 2, 64, F32, F32, TILED, 64, [perm[:5]], [16])
    # 2. bf16 fork tree: shared 3-page prefix, private tails, partial last pages,
    #    an INVALID id inside one table, an empty table.
    pre = perm[5:8]
    t2 = [pre + perm[8:10], pre + perm[10:12], pre + [INVALID] + perm[12:13], [], pre]
    case(s, "bf16_tree", 2, 8, 2, 64, BF16, BF16, TILED, 64, t2, [7, 16, 1, 0, 12])
    # 3. f16, interleaved GQA
    t3 = [perm[13:16], perm[13:15] + perm[16:18], perm[18:19]]
    case(s, "f16_interleaved", 3, 8, 4, 64, F16, F16, INTERLEAVED, 64, t3, [16, 9, 3])
    # 4. FP8 E4M3 with per (page, plane, head) f32 scales
    t4 = [perm[19:23], perm[19:21] + perm[23:25], perm[25:27]]
    case(s, "fp8_block", 4, 8, 2, 128, BF16, FP8, TILED, 64, t4, [5, 16, 11])
    # 5. MXFP8 with 20-sigma outliers (1 in 100)
    t5 = [perm[27:31], perm[27:30] + perm[31:32], perm[32:34]]
    case(s, "mxfp8_outliers", 5, 8, 2, 128, BF16, MX, TILED, 64, t5, [16, 2, 14], outlier_every=100)
    # 6. d = 256, one KV head for four query heads
    t6 = [perm[34:37], perm[34:35] + perm[37:38]]
    case(s, "bf16_d256", 6, 4, 1, 256, BF16, BF16, TILED, 64, t6, [16, 13])
    # 7. a single token: the output is that token's V row
    case(s, "f32_one_token", 7, 4, 2, 64, F32, F32, TILED, 64, [perm[38:39]], [1])
    np.savez_compressed(os.path.join(HERE, "decode_cases.npz"), **s)


if __name__ == "__main__":
    torch.manual_seed(0)
    tables()
    decode_cases()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
