"""dendrite_amd — MI355X (gfx950) paged tree-decode attention for Dendrite.

The compute lives in libdendrite_hip.so (C ABI: include/dendrite_hip.h),
hand-written HIP kernels plus a C++ host layer.  This package is the Python
host side over that ABI: the AttentionBackend mirror (HipBackend), the raw
pool / plan / decode calls, the block model, and the benchmark workloads.
"""
from ._lib import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, GQA_INTERLEAVED, GQA_TILED, INVALID_PAGE,
                   KV_BF16, KV_F16, KV_F32, KV_FP8_E4M3, KV_MXFP8, MAX_SEQ_LEN, PAGE_SIZE, DhError,
                   lib)
from .backend import (AttentionConfig, Backend, DecodePlan, HipBackend, Pool, decode_batch,
                      is_available)
from .cache import (BlockId, BlockPool, BlockTable, ForkHandle, KvCache, KvCacheConfig, NodeId,
                    NodeInfo, TreeState)

__all__ = [
    "AttentionConfig", "Backend", "BlockId", "BlockPool", "BlockTable", "DecodePlan", "DhError",
    "ForkHandle", "HipBackend", "KvCache", "KvCacheConfig", "NodeId", "NodeInfo", "Pool",
    "TreeState", "decode_batch", "is_available", "lib", "DTYPE_BF16", "DTYPE_F16", "DTYPE_F32",
    "GQA_INTERLEAVED", "GQA_TILED", "INVALID_PAGE", "KV_BF16", "KV_F16", "KV_F32", "KV_FP8_E4M3",
    "KV_MXFP8", "MAX_SEQ_LEN", "PAGE_SIZE",
]
