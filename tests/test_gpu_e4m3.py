"""The gfx950 e4m3 conversion (v_cvt_pk_fp8_f32) every quantiser uses,
against the software round-to-nearest-even conversion over all 2^32 fp32
bit patterns after the clamp, in every byte position of the packed word;
and against torch's float8_e4m3fn cast on a sample of the clamped range
through the library's own quantiser at scale 1."""

import numpy as np
import pytest
import torch

from helpers import np_u8

pytestmark = pytest.mark.gpu


def test_hardware_conversion_equals_software_for_every_fp32_pattern(device):
    from drama3_amd import _lib

    result = torch.tensor([0, -1], dtype=torch.int32, device=device)  # {count, first bad}
    chunk = 1 << 28
    for start in range(0, 1 << 32, chunk):
        _lib.call("d3_check_e4m3_conversion", start, chunk, result.data_ptr(),
                  _lib.stream(device))
    torch.cuda.synchronize()
    count, first_bad = (int(v) & 0xffffffff for v in result.cpu().tolist())
    assert count == 0, f"{count} mismatches, first at fp32 pattern {first_bad:#010x}"


def test_quantiser_at_unit_scale_equals_torch_cast(device):
    """A row whose largest magnitude is 448 has scale exactly 1, so its codes
    are the conversion of the values themselves: compare with torch."""
    from drama3_amd.moe_input import quantize_groups

    rng = np.random.default_rng(30)
    rows = 1 << 15
    bits = rng.integers(0, 0x43E00001, (rows, 128), dtype=np.uint32)  # |x| <= 448
    bits |= (rng.integers(0, 2, (rows, 128), dtype=np.uint32) << 31)
    bits[:, 0] = 0x43E00000  # 448.0: the row's scale is 448 / 448 = 1
    x = bits.view(np.float32)
    # the quantiser takes bf16 rows: keep the bf16-representable patterns
    x_bf16 = torch.from_numpy(x).to(torch.bfloat16)
    q, scales = quantize_groups(x_bf16.to(device))
    torch.cuda.synchronize()
    assert torch.all(scales.cpu() == 1.0)
    want = x_bf16.float().clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(np_u8(q.view(torch.uint8)), want)
