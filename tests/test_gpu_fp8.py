"""The kernels' in-register FP8 dequantisation, all 256 E4M3 codes, on the GPU,
against the oracle's OCP closed form (which tests/test_oracle.py pins against
torch.float8_e4m3fn)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from dendrite_amd import _lib

pytestmark = pytest.mark.gpu


def _bf16_to_f64(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("e8m0", [127, 123, 120, 116, 130, 134])
def test_e4m3_to_bf16_all_codes(e8m0):
    codes = np.arange(256, dtype=np.uint8)
    scales = np.full(64, e8m0, dtype=np.uint8)
    out = np.zeros(256, dtype=np.uint16)
    _lib.check(_lib.lib().dh_debug_e4m3_to_bf16(0, codes.ctypes.data_as(C.c_void_p),
                                                scales.ctypes.data_as(C.c_void_p), 256,
                                                out.ctypes.data_as(C.c_void_p)))
    got = _bf16_to_f64(out)
    want = np.array([oracle.e4m3_to_float(int(c)) for c in codes]) * 2.0 ** (e8m0 - 127)
    nan = np.isnan(want)
    bad = [(int(c), got[c], want[c]) for c in range(256)
           if not nan[c] and got[c] != want[c]]
    assert not bad, f"scale 2^{e8m0 - 127}: {len(bad)} codes differ, e.g. {bad[:6]}"
    assert np.all(np.isnan(got[nan])), "NaN codes must stay NaN"
