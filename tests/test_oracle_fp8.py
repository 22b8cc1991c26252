"""Pins the oracle's number formats and per-row quant (CPU only) against torch's own casts.

The oracle encodes e4m3 by searching the code table and bf16 by comparing neighbours; torch's float8_e4m3fn and
bfloat16 casts are the library routines the reference's quant numerics are defined by
(kernels/r9k_moe_mxfp4a8.hip:1729-1741; Appendix A of the reference's own quant contract)."""
import numpy as np
import torch

from oracle import oracle as O


def torch_e4m3_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_table_closed_form():
    t = O.e4m3_table()
    # OCP e4m3fn: 0x08 is the smallest normal 2^-6, 0x01 the smallest subnormal 2^-9, 0x7e the largest finite 448
    assert t[0x01] == 2.0 ** -9 and t[0x08] == 2.0 ** -6 and t[0x7e] == 448.0 and t[0x38] == 1.0
    assert np.isnan(t[0x7f]) and np.isnan(t[0xff]) and t[0x80] == 0.0 and np.signbit(t[0x80])
    assert np.all(np.diff(t[:0x7f]) > 0)


def test_e4m3_encode_all_bf16_patterns():
    """Every bf16 bit pattern (as fp32): the oracle's encode == torch's cast, NaNs compared as the NaN code."""
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    got = O.f32_to_e4m3(x)
    ref = torch_e4m3_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7f) == 0x7f)


def test_e4m3_encode_ties_and_range():
    """Exact midpoints between neighbouring codes (ties to even), one ulp either side, and the overflow edge."""
    t = O.e4m3_table()
    vals = []
    for c in range(0x7e):
        mid = np.float32((t[c] + t[c + 1]) / 2)
        vals += [mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9))]
    vals += [448.0, 460.0, 464.0, np.nextafter(np.float32(464.0), np.float32(1e9)), 479.0, 480.0, 1e30, 0.0, -0.0,
             2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11]
    x = np.array(vals, dtype=np.float32)
    x = np.concatenate([x, -x])
    assert np.array_equal(O.f32_to_e4m3(x), torch_e4m3_bits(x))


def test_e4m3_encode_random():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200000) * np.exp2(rng.uniform(-14, 9, 200000))).astype(np.float32)
    x = np.clip(x, -470, 470)
    assert np.array_equal(O.f32_to_e4m3(x), torch_e4m3_bits(x))


def test_bf16_encode_matches_torch():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(20000) * np.exp2(rng.uniform(-30, 30, 20000))).astype(np.float32)
    # exact ties: bf16 value + half a bf16 ulp
    b = (rng.integers(0, 1 << 15, 2000).astype(np.uint32) << 16) | 0x8000
    x = np.concatenate([x, b.view(np.float32), np.array([0.0, -0.0, 3.3895e38, 3.39e38], dtype=np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16(x)
    nan = np.isnan(x)                           # NaN payloads are not part of the contract: NaN stays NaN
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7f80) == 0x7f80) and np.all((got[nan] & 0x7f) != 0)


def _torch_quant(x: torch.Tensor):
    xf = x.float()
    amax = xf.abs().amax(-1).clamp_min(1e-12)
    # an IEEE division, as the reference kernel's `448.f / amax` (torch's `448.0 / tensor` is reciprocal * 448)
    inv = torch.div(torch.full_like(amax, 448.0), amax)
    q = (xf * inv[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q, (amax / 448.0).numpy()


def test_quant_rows_matches_torch():
    g = torch.Generator().manual_seed(3)
    for M, K, scale in ((16, 2048, 1.0), (7, 4096, 30.0), (3, 5120, 1e-3), (5, 96, 1.0)):
        x = (torch.randn(M, K, generator=g) * scale).to(torch.bfloat16)
        q, s = O.quant_rows_fp8(x)
        qr, sr = _torch_quant(x)
        assert np.array_equal(q, qr), (M, K)
        assert np.array_equal(s.view(np.uint32), sr.astype(np.float32).view(np.uint32)), (M, K)


def test_quant_rows_edge_rows():
    """All-zero row (amax clamps to 1e-12), one huge value, tiny values rounding to (negative) zero."""
    x = torch.zeros(4, 64)
    x[1, 3] = 3.0e38
    x[1, 4] = -1.0
    x[2] = torch.linspace(-1e-3, 1e-3, 64)
    x[2, 0] = 5.0
    x[3] = -1e-30
    x[3, 7] = 1.0
    x = x.to(torch.bfloat16)
    q, s = O.quant_rows_fp8(x)
    qr, sr = _torch_quant(x)
    assert np.array_equal(q, qr)
    assert np.array_equal(s, sr.astype(np.float32))
    assert np.all(q[0] == 0) and s[0] == np.float32(np.float32(1e-12) / np.float32(448.0))
    assert q[3, 0] == 0x80                      # a negative value that rounds to zero keeps the sign
