"""The device FP32 -> BF16 rounding every kernel stores with (gfx950's v_cvt_pk_bf16_f32) against the reference's
integer round-to-nearest-even (strixite common/bf16.hpp:19-26, restated as oracle.f32_to_bf16), bit for bit: random
bit patterns over the whole FP32 range, ties at every exponent, denormals, infinities and NaN payloads."""
import numpy as np
import pytest
import torch

import oracle as orc
from strixite_amd import _lib as L

pytestmark = pytest.mark.gpu


def test_device_bf16_rounding_is_integer_rne():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    e = np.arange(256, dtype=np.uint32) << 23
    ties = np.concatenate([e | 0x8000, e | 0x18000, e | 0x7FFF, e | 0x17FFF, e | 0x8001])  # halfway, +-1 ulp
    special = np.array([0, 0x80000000, 1, 0x807FFFFF, 0x7F800000, 0xFF800000, 0x7F800001, 0x7FC00000, 0xFFFFFFFF,
                        0x7F7FFFFF, 0x7F7F8000, 0x00008000, 0x00018000], np.uint32)
    allbits = np.concatenate([bits, ties, ties | 0x80000000, special])
    x = torch.from_numpy(allbits.view(np.float32)).cuda()
    y = torch.empty(x.numel(), dtype=torch.int16, device="cuda")
    assert L.lib().strix_calib_bf16_round(x.data_ptr(), y.data_ptr(), x.numel(), None) == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.uint16)
    want = orc.f32_to_bf16(allbits.view(np.float32))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(allbits[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
