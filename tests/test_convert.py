"""mft_convert on the GPU against the oracle's conversions, bit for bit.

fp32 -> bf16 is the reference's rounding (core/dtype.h:114-121,
float32_to_bf16_bits: add 0x7FFF plus the kept lsb, keep the high half; the
oracle's to_bf16_bits is pinned to the reference's own function in
test_oracle.py).  bf16 -> fp32 is exact (core/dtype.h:123-128).  The inputs
hold ties (both parities of the kept lsb), values one ulp either side of a
tie, signed zeros, subnormals, the largest finite floats (which round to
infinity), infinities and NaNs with payloads in either half; lengths cover
the 8-element vector body and its tail.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _specials():
    u = np.array([
        0x00000000, 0x80000000,              # +-0
        0x00000001, 0x807FFFFF, 0x00008000,  # subnormals (one a tie)
        0x3F808000, 0x3F818000,              # ties: kept lsb 0 and 1
        0x3F807FFF, 0x3F808001,              # one ulp either side of a tie
        0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF,  # max finite (rounds to inf), just below
        0x7F800000, 0xFF800000,              # +-inf
        0x7FC00000, 0x7F800001, 0x7FBFFFFF,  # NaNs: quiet, low payload, high payload
        0xFFFF0000, 0xFFFFFFFF,              # negative NaNs
    ], dtype=np.uint32)
    return u.view(np.float32)


def _inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32) * np.float32(1e3)
    bits = x.view(np.uint32)
    if n >= 4:  # force exact ties into a quarter of the values
        bits[: n // 4] = (bits[: n // 4] & 0xFFFF0000) | 0x8000
    sp = _specials()
    x[: min(n, sp.size)] = sp[: min(n, sp.size)]
    return x


@pytest.mark.parametrize("n", [1, 7, 8, 9, 19, 1000, 4096 * 257 + 5])
def test_f32_to_bf16_matches_reference_rounding(dev, orc, n):
    import torch
    from mobilefinetuner_amd import capi
    x = _inputs(n, seed=n)
    src = torch.from_numpy(x).to(dev)
    dst = torch.full((n,), 0x5A5A, dtype=torch.int16, device=dev)
    capi.convert(src.data_ptr(), capi.MFT_F32, dst.data_ptr(), capi.MFT_BF16, n,
                 torch.cuda.current_stream().cuda_stream)
    got = dst.cpu().numpy().view(np.uint16)
    want = orc.to_bf16_bits(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(x.view(np.uint32)[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


@pytest.mark.parametrize("n", [1, 8, 13, 1 << 20])
def test_bf16_to_f32_is_exact(dev, n):
    import torch
    from mobilefinetuner_amd import capi
    bits = np.random.default_rng(n).integers(0, 1 << 16, size=n, dtype=np.uint16)
    bits[: min(n, 4)] = np.array([0x0000, 0x8000, 0x7F80, 0x7FC1], np.uint16)[: min(n, 4)]
    src = torch.from_numpy(bits.view(np.int16)).to(dev)
    dst = torch.full((n,), 7.0, dtype=torch.float32, device=dev)
    capi.convert(src.data_ptr(), capi.MFT_BF16, dst.data_ptr(), capi.MFT_F32, n,
                 torch.cuda.current_stream().cuda_stream)
    got = dst.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, bits.astype(np.uint32) << 16)


def test_convert_rejects_bad_arguments(dev):
    import torch
    from mobilefinetuner_amd import capi
    a = torch.zeros(64, dtype=torch.float32, device=dev)
    b = torch.zeros(64, dtype=torch.int16, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    capi.convert(a.data_ptr(), capi.MFT_F32, b.data_ptr(), capi.MFT_BF16, 0, s)  # n = 0: nothing to do
    for args in [(a.data_ptr() + 4, capi.MFT_F32, b.data_ptr(), capi.MFT_BF16, 8),   # misaligned
                 (a.data_ptr(), capi.MFT_F32, b.data_ptr(), capi.MFT_F32, 8),        # same dtype
                 (a.data_ptr(), capi.MFT_F32, b.data_ptr(), capi.MFT_BF16, -1),      # negative n
                 (None, capi.MFT_F32, b.data_ptr(), capi.MFT_BF16, 8)]:
        with pytest.raises(capi.MftError):
            capi.convert(*args, s)
