"""Pins the oracle's top-k sum and dequant-then-matmul GEMM (CPU only).

moe_sum: a sequential fp32 loop (kernels/r9k_moe_sum.hip:37-55 of the reference) and, where every partial sum is
exact, torch's own bf16 sum. GEMM: pure-Python dot products on tiny inputs against oracle.grouped_gemm, and the
MXFP4 dequant against the E2M1 x 2^(e - 127) closed form (the reference tests' mx_deq)."""
import numpy as np
import torch

from helpers import make_experts
from oracle import oracle as O


def test_moe_sum_sequential_loop():
    g = torch.Generator().manual_seed(0)
    down = (torch.randn(3, 8, 64, generator=g) * 0.5).to(torch.bfloat16)
    shared = (torch.randn(3, 64, generator=g) * 0.5).to(torch.bfloat16)
    for sh in (None, shared):
        got = O.moe_sum(down, sh)
        d = down.float().numpy()
        for m in range(3):
            for n in range(64):
                acc = np.float32(0)
                for j in range(8):
                    acc = np.float32(acc + d[m, j, n])
                if sh is not None:
                    acc = np.float32(acc + sh.float().numpy()[m, n])
                ref = torch.tensor([acc]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)[0]
                assert got[m, n] == ref


def test_moe_sum_exact_sums_match_torch():
    g = torch.Generator().manual_seed(1)
    down = (torch.randint(-64, 64, (5, 8, 256), generator=g).float() / 16).to(torch.bfloat16)
    ref = down.float().sum(1).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.moe_sum(down), ref)


def test_mxfp4_dequant_closed_form():
    p = torch.tensor([[[0x10, 0xf7] + [0] * 14]], dtype=torch.uint8)          # codes 0,1,7,15, then zeros
    e = torch.tensor([[[127]]], dtype=torch.uint8)
    v = O.mxfp4_dequant(p, e)[0, 0]
    assert v[:4].tolist() == [0.0, 0.5, 6.0, -6.0]
    e = torch.tensor([[[120]]], dtype=torch.uint8)
    assert O.mxfp4_dequant(p, e)[0, 0, 2].item() == 6.0 * 2.0 ** -7


def test_grouped_gemm_python_loop():
    g = torch.Generator().manual_seed(2)
    E, N, K, T, k = 3, 16, 64, 4, 2
    packed, e8 = make_experts(E, N, K, g, 120, 130)
    W = {e: O.mxfp4_dequant(packed[e], e8[e]) for e in range(E)}
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    xq, xs = O.quant_rows_fp8(x)
    ids = np.array([[0, 2], [1, 0], [2, 1], [0, 1]], dtype=np.int32)
    tw = np.array([0.25, 0.75, 0.5, 0.5, 0.1, 0.9, 0.6, 0.4], dtype=np.float32)
    out = O.grouped_gemm(xq, xs, W, ids.reshape(-1), k, tw)
    tab = O.e4m3_table()
    for r in range(T * k):
        t, e = r // k, int(ids.reshape(-1)[r])
        for n in range(N):
            acc = sum(tab[xq[t, kk]] * float(W[e][n, kk]) for kk in range(K))
            sc = np.float32(np.float32(xs[t]) * np.float32(tw[r]))
            v = np.float32(np.float32(acc) * sc)
            ref = torch.tensor([v]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)[0]
            assert out[r, n] == ref


def test_router_gemm_python_loop():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 24, generator=g).to(torch.bfloat16)
    w = torch.randn(5, 24, generator=g).to(torch.bfloat16)
    ref = O.router_gemm(x, w)
    xf, wf = x.double().tolist(), w.double().tolist()
    for m in range(3):
        for e in range(5):
            assert ref[m, e].item() == sum(a * b for a, b in zip(xf[m], wf[e]))


def test_hc_silu_epilogue():
    v = torch.tensor([[0.0, 3.0, -40.0, 40.0, 1.0078125, 2.5]], dtype=torch.float32)
    hc = 2.0
    out = O.hc_silu(v, 5, hc)
    s = v.to(torch.bfloat16).double() / hc
    assert torch.allclose(out[:, :5], torch.nn.functional.silu(s)[:, :5], rtol=1e-15, atol=0)
    assert out[0, 0] == 0.0 and abs(out[0, 2]) < 1e-7 and abs(out[0, 3] - 20.0) < 1e-7    # silu(0), the limits
    assert out[0, 5] == 2.5                                                                # past act_cols: v
    # s is taken from the bf16-rounded v: 1.0078125 is bf16-exact, 1.00390625 rounds to 1.0 (tie to even)
    assert O.hc_silu(torch.tensor([[1.00390625]]), 1, 1.0)[0, 0] == O.hc_silu(torch.tensor([[1.0]]), 1, 1.0)[0, 0]


def test_nvfp4_gemm_python_loop():
    """The native NVFP4 GEMM against dot products over the closed-form code values (e2m1 table, e4m3 exponent /
    mantissa), the multiplier and the row scale applied in the kernel's order, on a tiny routed case."""
    rng = np.random.default_rng(5)
    E, N, Kd, R = 2, 3, 32, 3
    packed = rng.integers(0, 256, (E, N, Kd // 2), dtype=np.uint8)
    s16 = rng.integers(0, 0x7f, (E, N, Kd // 16), dtype=np.uint8)       # finite e4m3 codes, subnormals included
    wg = rng.uniform(0.5, 2.0, (E, N)).astype(np.float32)
    aq = rng.integers(0, 256, (R, Kd), dtype=np.uint8)
    aq[(aq & 0x7f) == 0x7f] = 0                                          # no NaN codes
    a_s = rng.uniform(0.01, 0.1, R).astype(np.float32)
    tw = rng.uniform(0.1, 1.0, R).astype(np.float32)
    eor = np.array([1, 0, 1], dtype=np.int32)
    got = O.nvfp4_gemm(aq, a_s, packed, s16, wg, eor, 1, tw)

    def e2m1(c):
        m = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0][c & 7]
        return -m if c & 8 else m

    def e4m3(b):
        e, m = (b >> 3) & 15, b & 7
        v = (1 + m / 8) * 2.0 ** (e - 7) if e else m / 8 * 2.0 ** -6
        return -v if b & 0x80 else v

    for r in range(R):
        e = eor[r]
        for n in range(N):
            acc = 0.0
            for k in range(Kd):
                byte = int(packed[e, n, k // 2])
                code = byte & 15 if k % 2 == 0 else byte >> 4
                acc += e4m3(int(aq[r, k])) * e2m1(code) * e4m3(int(s16[e, n, k // 16]))
            sc = np.float32(np.float32(wg[e, n]) * np.float32(a_s[r])) * np.float32(tw[r])
            want = torch.tensor([np.float32(acc) * sc], dtype=torch.float32).to(torch.bfloat16)
            assert got[r, n] == O.bf16_bits(want)[0], (r, n)
