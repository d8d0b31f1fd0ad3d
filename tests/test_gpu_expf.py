"""The device build of the product's expf against the host libm, bit for bit,
on every non-positive float (softmax only ever evaluates exp(l - max) <= 0)
and on a strided sample of the positive ones."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
KIT = Path(__file__).resolve().parent / "cpp" / "libdevice_expf.so"


def test_device_expf_equals_libm():
    import torch
    L = ctypes.CDLL(str(KIT))
    L.device_expf_range.restype = ctypes.c_int
    L.device_expf_range.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    n = 1 << 26
    out = torch.empty(n, dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    bad = checked = 0
    starts = list(range(0x80000000, 0x100000000, n)) + [0x00000000, 0x3f800000, 0x42000000]
    for start in starts:
        m = min(n, 0x100000000 - start)
        assert L.device_expf_range(start, out.data_ptr(), m, stream) == 0
        bits = np.arange(start, start + m, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        want = O.expf_many(x)
        got = out[:m].cpu().numpy()
        nan = np.isnan(x)
        bad += int(np.count_nonzero(got.view(np.uint32)[~nan] != want.view(np.uint32)[~nan]))
        checked += int(np.count_nonzero(~nan))
    assert checked > 2_100_000_000
    assert bad == 0, f"{bad} of {checked} floats differ from libm expf"
