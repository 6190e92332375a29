"""The kernels' activation quantiser encodes on the conversion unit
(v_cvt_pk_fp8_f32 after a clamp to +-448, NaN kept as sign | 0x7f).  Over all
2^32 float bit patterns, in every byte position of the packed word, it must
give the codes of the software encoder that test_e4m3_encoder.py pins to the
oracle and to torch's float8_e4m3fn cast."""
import pytest
import torch

from conftest import say

pytestmark = pytest.mark.gpu


def test_hardware_encoding_equals_software_encoder_everywhere(lib, dev):
    bad = torch.zeros(1, dtype=torch.int64, device=dev)
    chunk = 1 << 28
    for c in range(16):
        lib.e4m3_check(c * chunk, chunk, bad)
    torch.cuda.synchronize()
    say(f"e4m3 check: {int(bad.item())} mismatching patterns of 2^32")
    assert int(bad.item()) == 0


def test_saturation_and_nan_ranges_and_counter_accumulates(lib, dev):
    """The ranges where an unclamped conversion would differ (448 and past
    464, infinities, NaNs) agree, and the counter is added to, not reset."""
    bad = torch.full((1,), 5, dtype=torch.int64, device=dev)
    lib.e4m3_check(0x43e00000, 1 << 20, bad)      # 448 .. well past 464
    lib.e4m3_check(0x7f800000, 1 << 20, bad)      # inf, NaNs
    torch.cuda.synchronize()
    assert int(bad.item()) == 5
