"""Pins the oracle's NVFP4 dequant and MSE-searched MXFP4 requant (CPU only).

The reference (r9700_vllm/quant/nvfp4.py:35-90) is torch code; the oracle restates it in C with different
formulations (nearest-value search, brute-force exponent, fp64 errors). Here each step is pinned by
  * the E2M1 closed form and torch.bucketize on the reference's thresholds (library routine),
  * brute force on the exponent rule and on the candidate choice,
  * a torch restatement in fp32 with torch.log2 / torch.bucketize (the reference's own operations), bit-exact on
    NVFP4-derived data, and agreement of fp32 ceil(log2(amax/6)) with the exact rule for every NVFP4-derivable
    block maximum,
  * the reference test's quality criterion (tests/test_nvfp4.py:47-59): conversion error < 1.05x the floor of two
    independent roundings."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

E2M1_T = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
MID_T = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])


def nvfp4_quant(w: torch.Tensor):
    """CT-style NVFP4 (the reference test's generator, tests/test_nvfp4.py:18-27): global divisor gd, e4m3 scale
    per 16, RTN E2M1. -> (packed u8 [N, K/2], s16 bytes [N, K/16], gd)."""
    N, K = w.shape
    gd = (448.0 * 6.0 / w.abs().max()).float()
    x = w.float().reshape(N, K // 16, 16)
    s16 = (x.abs().amax(-1) / 6.0 * gd).clamp(min=2 ** -9).to(torch.float8_e4m3fn)
    v = x * gd / s16.float().unsqueeze(-1)
    code = torch.bucketize(v.abs(), MID_T).to(torch.uint8) | ((v < 0).to(torch.uint8) << 3)
    code = code.reshape(N, K)
    return (code[:, 0::2] | (code[:, 1::2] << 4)).numpy(), s16.view(torch.uint8).numpy(), gd


def torch_search(w: torch.Tensor):
    """fp32 torch restatement with the reference's operations (log2, ceil, exp2, bucketize, fp32 sum)."""
    N, K = w.shape
    x = w.float().reshape(N, K // 32, 32)
    amax = x.abs().amax(-1, keepdim=True).clamp_min(2.0 ** -126)
    e0 = torch.ceil(torch.log2(amax / 6.0)).clamp(-126, 127)
    best = None
    for d in (0, -1):
        e = (e0 + d).clamp(-127, 127)
        s = torch.exp2(e)
        c = torch.bucketize((x / s).abs(), MID_T).to(torch.uint8) | (((x / s) < 0).to(torch.uint8) << 3)
        err = ((E2M1_T[c.long()] * s - x) ** 2).sum(-1, keepdim=True)
        if best is None:
            best = (c, e, err)
        else:
            take = err < best[2]
            best = (torch.where(take, c, best[0]), torch.where(take, e, best[1]), torch.minimum(err, best[2]))
    c = best[0].reshape(N, K)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).numpy(), (best[1].squeeze(-1) + 127).to(torch.uint8).numpy()


def mx_dequant(p: np.ndarray, e: np.ndarray) -> torch.Tensor:
    return O.mxfp4_dequant(torch.from_numpy(p), torch.from_numpy(e))


def test_e2m1_encode_matches_bucketize():
    grid = [0.0, 6.0, 7.5, 100.0, 0.1]
    for m in [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]:
        m32 = np.float32(m)
        grid += [m32, np.nextafter(m32, np.float32(0)), np.nextafter(m32, np.float32(10))]
    rng = np.random.default_rng(0)
    v = np.concatenate([np.array(grid, dtype=np.float32), rng.uniform(0, 8, 5000).astype(np.float32)])
    v = np.concatenate([v, np.array([np.inf], dtype=np.float32)])
    v = np.concatenate([v, -v, np.array([-0.0, -1e-30], dtype=np.float32)])
    lib = O.lib()
    got = np.array([lib.or_e2m1_encode(float(x)) for x in v], dtype=np.uint8)
    t = torch.from_numpy(v)
    ref = (torch.bucketize(t.abs(), MID_T).to(torch.uint8) | ((t < 0).to(torch.uint8) << 3)).numpy()
    assert np.array_equal(got, ref)
    assert got[-2] == 0 and got[-1] == 8       # -0.0 -> code 0; a negative value rounding to zero -> code 8


def test_exponent_rule_brute_force():
    rng = np.random.default_rng(1)
    a = np.exp2(rng.uniform(-126, 120, 4000)).astype(np.float32)
    a = np.concatenate([a, np.float32(6.0) * np.exp2(np.arange(-120, 120)).astype(np.float32)])
    lib = O.lib()
    for x in a:
        e = lib.or_exp_no_clip(float(x))
        assert np.ldexp(6.0, e) >= float(x) > np.ldexp(6.0, e - 1)


def test_fp32_log2_agrees_on_nvfp4_maxima():
    """For every block maximum an NVFP4 block with global scale 1 can have (E2M1 magnitude x e4m3 scale), the
    reference's fp32 ceil(log2(amax / 6)) equals the exact exponent rule used by the oracle and the kernel."""
    t = O.e4m3_table()
    lib = O.lib()
    mags = [0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    vals = sorted({np.float32(np.float32(m) * np.float32(t[b])) for m in mags for b in range(1, 0x7f)})
    for a in vals:
        a = max(a, np.float32(2.0 ** -126))
        ref = int(np.ceil(np.log2(np.float32(a) / np.float32(6.0), dtype=np.float32)))
        assert max(-126, min(127, ref)) == max(-126, min(127, lib.or_exp_no_clip(float(a))))


def test_search_brute_force_candidates():
    """The chosen exponent is the better of {e0, e0 - 1} by exact squared error (ties keep e0), and the codes are
    the nearest-value encodes at that exponent."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 256)) * np.exp2(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    w[0, :32] = 0.0                                    # all-zero block: e = -126, byte 1
    w[1, :32] = -0.0
    p, e = O.quantize_mxfp4_search(w)
    assert e[0, 0] == 1 and e[1, 0] == 1 and np.all(p[0, :16] == 0) and np.all(p[1, :16] == 0)
    lib = O.lib()
    for n in range(2, 64):
        for b in range(8):
            x = w[n, b * 32:(b + 1) * 32].astype(np.float64)
            amax = max(np.abs(x).max(), 2.0 ** -126)
            e0 = max(-126, min(127, lib.or_exp_no_clip(float(amax))))
            errs = []
            for cand in (e0, max(-127, e0 - 1)):
                c = np.array([lib.or_e2m1_encode(float(np.float32(v) / np.float32(2.0 ** cand))) for v in x])
                errs.append(((O.E2M1[c] * 2.0 ** cand - x) ** 2).sum())
            want = e0 if not errs[1] < errs[0] else max(-127, e0 - 1)
            assert int(e[n, b]) - 127 == want


@pytest.mark.parametrize("N,K", [(256, 512), (512, 2560), (64, 5120)])
def test_nvfp4_conversion_matches_torch_restatement(N, K):
    g = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, K, generator=g) * torch.exp(torch.randn(N, 1, generator=g) * 0.3) * 0.02
    p16, s16, gd = nvfp4_quant(w)
    div = np.full(N, np.float32(gd), dtype=np.float32)
    deq = O.dequant_nvfp4(p16, s16, div)
    # exact dequant == E2M1 closed form x e4m3 value / divisor, in fp32 (nvfp4.py:39-46)
    c = np.stack((p16 & 15, p16 >> 4), -1).reshape(N, K)
    ref = (E2M1_T.numpy()[c].reshape(N, -1, 16).astype(np.float32)
           * O.e4m3_table()[s16].astype(np.float32)[..., None]).reshape(N, K) / np.float32(gd)
    assert np.array_equal(deq, ref.astype(np.float32))
    pm, em = O.nvfp4_to_mxfp4(p16, s16, div)
    pt, et = torch_search(torch.from_numpy(deq))
    assert np.array_equal(pm, pt) and np.array_equal(em, et)
    # the reference test's criterion: within 1.05x the floor of two independent roundings
    conv = mx_dequant(pm, em)
    rtn_p, rtn_e = O.quantize_mxfp4_search(w.numpy())          # a direct MXFP4 of the original weights
    rel = lambda a, b: float((a.double() - b.double()).norm() / b.double().norm())
    wt = w.double()
    e_nv, e_conv = rel(torch.from_numpy(deq), wt), rel(conv, wt)
    e_rtn = rel(mx_dequant(rtn_p, rtn_e), wt)
    assert e_conv < 1.05 * (e_nv ** 2 + e_rtn ** 2) ** 0.5


def test_config4_scale_generator_roundtrip():
    """BASELINE config 4's NVFP4 form (codes uniform, s16 = e4m3(|N(0,1)| * 0.05), global 1): conversion equals the
    fp32 torch restatement bit for bit on a slice of the full shape."""
    g = torch.Generator().manual_seed(4)
    N, K = 128, 5120
    p16 = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8).numpy()
    s16 = (torch.randn(N, K // 16, generator=g).abs() * 0.05).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    div = np.ones(N, dtype=np.float32)
    pm, em = O.nvfp4_to_mxfp4(p16, s16, div)
    pt, et = torch_search(torch.from_numpy(O.dequant_nvfp4(p16, s16, div)))
    assert np.array_equal(pm, pt) and np.array_equal(em, et)


def _mismatches(w: torch.Tensor) -> tuple[int, int]:
    pm, em = O.quantize_mxfp4_search(w.numpy())
    pt, et = torch_search(w)
    N = w.shape[0]
    bad = (em != et) | (pm.reshape(N, -1, 16) != pt.reshape(N, -1, 16)).any(-1)
    return int(bad.sum()), bad.size


def test_search_matches_torch_restatement_on_arbitrary_fp32():
    """quantize_mxfp4_search (exact exponent rule, fp64 error sums) against the fp32 torch restatement
    (torch.log2, exp2, bucketize, fp32 sums: the reference's operations) on weights that are NOT NVFP4-derived:
      * wide-range random blocks (per-row magnitudes spread over ~6 binades);
      * block maxima 1..8 ulp above 6 * 2^k for k in [-100, 98], where fp32 ceil(log2(amax / 6)) can land one
        below the exact exponent -- the result still agrees, because both candidate pairs contain e = k and the
        coarser exponent never wins for a block whose maximum sits on 6 * 2^k;
      * the 2048 blocks (of 200K) whose two candidate errors are closest, exact ties included (ties keep e0 in both);
      * blocks holding +-inf next to finite values (bucketize puts inf past the last midpoint: code 6).
    The mismatch count is 0 on every set."""
    g = torch.Generator().manual_seed(11)
    wide = torch.randn(256, 2048, generator=g) * torch.exp(torch.randn(256, 1, generator=g) * 2)
    rng = np.random.default_rng(0)
    rows = []
    for k in range(-100, 100, 3):
        for d in range(1, 9):
            b = rng.standard_normal(32).astype(np.float32)
            b = (b / np.abs(b).max() * np.float32(3.0) * np.float32(2.0 ** k)).astype(np.float32)
            b[d] = np.float32(6.0 * 2.0 ** k) * np.float32(1 + d * 2.0 ** -23)
            rows.append(b)
    edge = torch.from_numpy(np.stack(rows[: len(rows) // 8 * 8]).reshape(-1, 256).copy())
    x = torch.randn(200000, 32, generator=g)
    e0 = torch.ceil(torch.log2(x.abs().amax(-1, keepdim=True) / 6))
    errs = []
    for d in (0, -1):
        s = torch.exp2(e0 + d)
        v = E2M1_T[torch.bucketize((x / s).abs(), MID_T)].double() * torch.sign(x).double() * s.double()
        errs.append(((v - x.double()) ** 2).sum(-1))
    near = x[torch.argsort(((errs[0] - errs[1]).abs() / errs[0]))[:2048]].reshape(-1, 256).contiguous()
    assert float(((errs[0] - errs[1]).abs() / errs[0]).min()) == 0.0      # the set really holds exact ties
    inf = torch.randn(8, 256, generator=g)
    inf[0, 3], inf[1, 40], inf[2, 7], inf[2, 9], inf[3, :32] = float("inf"), -float("inf"), float("inf"), -1e30, 0.0
    inf[3, 31] = -float("inf")
    for name, w in (("wide-range", wide), ("log2 edge", edge), ("near-tie", near), ("infinite", inf)):
        bad, n = _mismatches(w)
        print(f"{name}: {bad} of {n} blocks differ from the fp32 torch restatement", flush=True)
        assert bad == 0, name
