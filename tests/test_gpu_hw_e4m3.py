"""The gfx950 hardware e4m3 conversions against the library's encoder (torch's
float8_e4m3fn cast semantics, pinned in test_oracle.py), exhaustively: e4m3x4_clamped
(the MX quantizers, after their clamp to +-448) on every float32 of magnitude at most 448,
and e4m3x4_torch (the FP8 activation prologue: no clamp, the hardware result with
positive NaNs set to 0x7F) on every float32 bit pattern."""
import pytest
import torch

from vllm_quant_kernels import _lib

pytestmark = pytest.mark.gpu


def _mismatches(full: int):
    count = torch.zeros(1, dtype=torch.int32, device="cuda")
    first = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("vqk_debug_e4m3_hw_check", 0, 0x80000000 if full else 0x43E00001, full,
              count.data_ptr(), first.data_ptr(), st)
    _lib.call("vqk_debug_e4m3_hw_check", 0x80000000, 0xFFFFFFFF if full else 0xC3E00001, full,
              count.data_ptr(), first.data_ptr(), st)
    torch.cuda.synchronize()
    return int(count.item()), int(first.item()) & 0xFFFFFFFF


@pytest.mark.parametrize("full", [0, 1])
def test_hw_e4m3_equals_encoder(full):
    n, f = _mismatches(full)
    assert n == 0, f"{n} mismatches, first at 0x{f:08x}"
