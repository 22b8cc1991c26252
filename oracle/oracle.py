"""CPU oracle for the quantized-MoE hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker (or, in bench.py, as the timed CPU baseline). The product (r9700-stack_amd/) never imports it.

Integer / byte parts come from liboracle.so (oracle/r9k_oracle.c, built by oracle/Makefile): fp8 and bf16
encodes, per-row quant, routing ids, align tables, the top-k sum, NVFP4 -> MXFP4. The floating-point parts are the
reference's own dequant-then-matmul restated in torch on the CPU (tests/test_moe_mxfp4.py:16-72 and
kernels/r9k_moe_mxfp4a8.hip:469-482 of the reference fix the math and the rounding points): each GEMM output row is
bf16(acc * (As * topk_w)) with acc = dequant(A row) . dequant(W row) accumulated in fp64.

Parity status per function (what pins it; tests/test_oracle_*.py):
  e4m3 encode, quant_rows_fp8      torch float8_e4m3fn cast (library routine), exhaustive over bf16 inputs
  bf16 encode                      torch bfloat16 cast (library routine)
  silu_mul_quant_fp8               torch silu in fp32 (tolerance) + torch cast of the same products (exact)
  route                            torch.softmax + stable sort (ids exact, weights 2e-6), degenerate-row rules
  align                            numpy stable argsort restatement + the reference test's table invariants
  moe_sum                          sequential fp32 loop + exactly-representable sums vs torch
  nvfp4 dequant / search           E2M1 closed form, brute-force nearest value and exponent, the reference
                                   test's error-floor criterion, fp32-log2 agreement on all NVFP4-derivable maxima
  gemm / layer                     pure-Python dot products on tiny inputs
  router_gemm / hc_silu            pure-Python dot products; torch silu (library routine) and its closed-form limits
  nvfp4_gemm                       pure-Python dot products over the closed-form e2m1 / e4m3 values on tiny inputs
  lru_manage / lru_gather          a serial one-argmin-per-insert simulation written independently in the test,
                                   hand-worked step sequences, and the cache invariants (table / map_cold
                                   complementary, slot_expert inverse of table, no routed resident evicted)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(HERE, "_build", "liboracle.so")
_L = None

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                dtype=np.float64)


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return _SO


def lib() -> ctypes.CDLL:
    global _L
    if _L is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        i, l, f = ctypes.c_int, ctypes.c_long, ctypes.c_float
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [f]
        L.or_f32_to_e4m3.restype = ctypes.c_uint8
        L.or_f32_to_e4m3.argtypes = [f]
        L.or_e4m3_value.restype = ctypes.c_double
        L.or_e4m3_value.argtypes = [ctypes.c_uint8]
        L.or_f32_to_e4m3_array.argtypes = [P, P, l]
        L.or_quant_rows_fp8.argtypes = [P, i, i, l, P, P]
        L.or_silu_mul_quant_fp8.argtypes = [P, i, i, P, P, P]
        L.or_moe_route.restype = i
        L.or_moe_route.argtypes = [P, l, i, i, i, i, P, P]
        L.or_moe_align.restype = i
        L.or_moe_align.argtypes = [P, l, i, i, P, P, P]
        L.or_capacity.restype = l
        L.or_capacity.argtypes = [l, i, i]
        L.or_moe_sum.argtypes = [P, P, P, i, i, i, l, l]
        L.or_e2m1_encode.restype = ctypes.c_uint8
        L.or_e2m1_encode.argtypes = [f]
        L.or_exp_no_clip.restype = i
        L.or_exp_no_clip.argtypes = [f]
        L.or_dequant_nvfp4.argtypes = [P, P, P, i, i, P]
        L.or_quantize_mxfp4_search.argtypes = [P, i, i, P, P]
        L.or_nvfp4_to_mxfp4.argtypes = [P, P, P, i, i, P, P]
        _L = L
    return _L


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> uint16 numpy bits."""
    return np.ascontiguousarray(x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def bits_to_bf16(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


_E4M3 = None


def e4m3_table() -> np.ndarray:
    """float64 value of every e4m3fn byte (NaN for 0x7f / 0xff)."""
    global _E4M3
    if _E4M3 is None:
        L = lib()
        _E4M3 = np.array([L.or_e4m3_value(b) for b in range(256)], dtype=np.float64)
    return _E4M3


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.uint8)
    lib().or_f32_to_e4m3_array(_p(x), _p(q), x.size)
    return q


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return np.array([L.or_f32_to_bf16(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


# ------------------------------------------------------------------------------------------ activations
def quant_rows_fp8(x: torch.Tensor):
    """bf16 [M, K] -> (q uint8 [M, K], s float32 [M])."""
    xb = bf16_bits(x)
    M, K = xb.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().or_quant_rows_fp8(_p(xb), M, K, K, _p(q), _p(s))
    return q, s


def silu_mul_quant_fp8(gu: torch.Tensor):
    """bf16 [M, 2I] -> (q uint8 [M, I], s float32 [M], act float32 [M, I])."""
    gb = bf16_bits(gu)
    M, I2 = gb.shape
    I = I2 // 2
    q = np.empty((M, I), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    act = np.empty((M, I), dtype=np.float32)
    lib().or_silu_mul_quant_fp8(_p(gb), M, I, _p(q), _p(s), _p(act))
    return q, s, act


# ------------------------------------------------------------------------------------- routing and tables
def route(logits: torch.Tensor, topk: int, renorm: bool):
    """bf16 [M, E] -> (w float32 [M, topk], ids int32 [M, topk])."""
    lb = bf16_bits(logits)
    M, E = lb.shape
    w = np.empty((M, topk), dtype=np.float32)
    ids = np.empty((M, topk), dtype=np.int32)
    rc = lib().or_moe_route(_p(lb), E, M, E, topk, 1 if renorm else 0, _p(w), _p(ids))
    if rc:
        raise ValueError(f"or_moe_route rejected M={M} E={E} topk={topk}")
    return w, ids


def capacity(numel: int, E: int, blk: int) -> int:
    return int(lib().or_capacity(numel, E, blk))


def align(ids: np.ndarray, E: int, blk: int):
    """ids int [numel] -> (sorted_ids [cap], expert_ids [cap/blk], ntpp [1]) int32, canonical order."""
    flat = np.ascontiguousarray(np.asarray(ids).reshape(-1), dtype=np.int32)
    numel = flat.size
    cap = capacity(numel, E, blk)
    s = np.empty(cap, dtype=np.int32)
    e = np.empty(cap // blk, dtype=np.int32)
    n = np.empty(1, dtype=np.int32)
    lib().or_moe_align(_p(flat), numel, E, blk, _p(s), _p(e), _p(n))
    return s, e, n


def moe_sum(down: torch.Tensor, shared: torch.Tensor | None = None) -> np.ndarray:
    """bf16 [M, topk, N] (+ bf16 [M, N]) -> uint16 bf16 bits [M, N]."""
    db = bf16_bits(down)
    M, topk, N = db.shape
    out = np.empty((M, N), dtype=np.uint16)
    sb = bf16_bits(shared) if shared is not None else None
    lib().or_moe_sum(_p(db), _p(sb) if sb is not None else None, _p(out), M, topk, N, N, N)
    return out


# ------------------------------------------------------------------------------------------- NVFP4 / MXFP4
def dequant_nvfp4(packed: np.ndarray, s16: np.ndarray, row_div: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    s16 = np.ascontiguousarray(s16, dtype=np.uint8)
    row_div = np.ascontiguousarray(row_div, dtype=np.float32)
    N, Kh = packed.shape
    out = np.empty((N, Kh * 2), dtype=np.float32)
    lib().or_dequant_nvfp4(_p(packed), _p(s16), _p(row_div), N, Kh * 2, _p(out))
    return out


def quantize_mxfp4_search(w: np.ndarray):
    """fp32 [N, K] -> (packed uint8 [N, K/2], e8m0 uint8 [N, K/32])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    p = np.empty((N, K // 2), dtype=np.uint8)
    e = np.empty((N, K // 32), dtype=np.uint8)
    lib().or_quantize_mxfp4_search(_p(w), N, K, _p(p), _p(e))
    return p, e


def nvfp4_to_mxfp4(packed: np.ndarray, s16: np.ndarray, row_div: np.ndarray):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    s16 = np.ascontiguousarray(s16, dtype=np.uint8)
    row_div = np.ascontiguousarray(row_div, dtype=np.float32)
    N, Kh = packed.shape
    p = np.empty((N, Kh), dtype=np.uint8)
    e = np.empty((N, Kh * 2 // 32), dtype=np.uint8)
    lib().or_nvfp4_to_mxfp4(_p(packed), _p(s16), _p(row_div), N, Kh * 2, _p(p), _p(e))
    return p, e


_LUT2 = None


def mxfp4_dequant(packed: torch.Tensor, e8m0: torch.Tensor, dtype=torch.float64) -> torch.Tensor:
    """[..., N, K/2] codes + [..., N, K/32] exponents -> [..., N, K] values E2M1[c] * 2^(e - 127)
    (the reference tests' mx_deq: tests/test_fold_mxfp4.py:36-39, tests/test_prefill_4bit.py:19-22). One gather
    through a byte -> (even, odd) value table; exact in fp32 for exponent bytes below 253."""
    global _LUT2
    if _LUT2 is None:
        b = np.arange(256)
        _LUT2 = torch.from_numpy(np.stack([E2M1[b & 15], E2M1[b >> 4]], axis=1))     # [256, 2] float64
    v = _LUT2.to(dtype)[packed.to(torch.int64)]                                       # [..., N, K/2, 2]
    shape = (*packed.shape[:-1], packed.shape[-1] * 2)
    v = v.reshape(*packed.shape[:-1], -1, 32)
    sc = torch.exp2(e8m0.to(dtype) - 127.0).unsqueeze(-1)
    return (v * sc).reshape(shape)


def e4m3_dequant(q: np.ndarray, dtype=torch.float64) -> torch.Tensor:
    return torch.from_numpy(e4m3_table()[np.asarray(q, dtype=np.uint8)]).to(dtype)


# ------------------------------------------------------------------------------------------ GEMM / layer
def grouped_gemm(aq: np.ndarray, a_s: np.ndarray, w_deq, expert_of_row: np.ndarray, a_row_div: int,
                 topk_w: np.ndarray | None = None, rows: np.ndarray | None = None,
                 acc_dtype=torch.float64) -> np.ndarray:
    """bf16 bits [R, N] of out[r] = bf16((deq(aq[r // a_row_div]) . W[e_r]^T) * (a_s[r // a_row_div] * topk_w[r]))
    for the routed rows `rows` (default all). w_deq: expert -> dequantized [N, K] weight (a dict or a callable,
    evaluated one expert at a time). acc_dtype: fp64 (exact products, the GEMM parity tests) or fp32 (the
    fp32-accumulated layer reference). The scale product order and the single bf16 rounding follow
    kernels/r9k_moe_mxfp4a8.hip:478-481 of the reference."""
    get = w_deq if callable(w_deq) else (lambda e: w_deq[e])
    rows = np.arange(expert_of_row.size) if rows is None else np.asarray(rows)
    eor = expert_of_row[rows]
    out = None
    for e in np.unique(eor):
        sel = np.nonzero(eor == e)[0]
        r = rows[sel]
        W = get(int(e)).to(acc_dtype)
        if out is None:
            out = np.zeros((rows.size, W.shape[0]), dtype=np.uint16)
        a = e4m3_dequant(aq[r // a_row_div], acc_dtype)
        acc = (a @ W.T).to(torch.float32)
        sc = torch.from_numpy(a_s[r // a_row_div].astype(np.float32))
        if topk_w is not None:
            sc = sc * torch.from_numpy(topk_w[r].astype(np.float32))
        out[sel] = bf16_bits((acc * sc[:, None]).to(torch.bfloat16))
    return out


def nvfp4_gemm(aq: np.ndarray, a_s: np.ndarray, packed: np.ndarray, s16: np.ndarray, wg: np.ndarray,
               expert_of_row: np.ndarray, a_row_div: int, topk_w: np.ndarray | None = None,
               rows: np.ndarray | None = None) -> np.ndarray:
    """bf16 bits [R, N] of the native NVFP4 grouped GEMM for the routed rows `rows` (default all):
    out[r, n] = bf16(acc * ((wg[e, n] * a_s[r // d]) * topk_w[r])), acc = deq(aq[r // d]) . (e2m1 * s16)[e, n, :] in
    fp64 -- the reference's native path: exact e2m1 x e4m3 weights (kernels/r9k_moe_mxfp4a8.hip:89-96, 300-340), the
    per-row fp32 multiplier and the row scale in the epilogue in that order (:469-482). packed [E, N, K/2] u8,
    s16 [E, N, K/16] e4m3 bits, wg [E, N] fp32."""
    rows = np.arange(expert_of_row.size) if rows is None else np.asarray(rows)
    eor = expert_of_row[rows]
    E, N, Kh = packed.shape
    out = np.zeros((rows.size, N), dtype=np.uint16)
    for e in np.unique(eor):
        sel = np.nonzero(eor == e)[0]
        r = rows[sel]
        W = torch.from_numpy(dequant_nvfp4(packed[e], s16[e], np.ones(N, dtype=np.float32))).double()
        a = e4m3_dequant(aq[r // a_row_div], torch.float64)
        acc = (a @ W.T).to(torch.float32)
        sc = torch.from_numpy(wg[e].astype(np.float32))[None, :] * torch.from_numpy(
            a_s[r // a_row_div].astype(np.float32))[:, None]
        if topk_w is not None:
            sc = sc * torch.from_numpy(topk_w[r].astype(np.float32))[:, None]
        out[sel] = bf16_bits((acc * sc).to(torch.bfloat16))
    return out


def router_gemm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Router logits [M, E] = x [M, K] . w [E, K]^T from the bf16 values, accumulated in fp64 (the gate GEMM the
    reference's router kernel computes, kernels/r9k_router.hip:120-155; its test measures against this fp64 product,
    tests/test_router_r9k.py:50-56)."""
    return x.detach().cpu().double() @ w.detach().cpu().double().t()


def hc_silu(v: torch.Tensor, act_cols: int, hc: float) -> torch.Tensor:
    """The router kernel's hyper-connection epilogue (kernels/r9k_router.hip:34-40): columns < act_cols become
    s * sigmoid(s) with s = bf16(v) / hc; the others keep v. fp64 from the fp32 GEMM values v."""
    v = v.detach().cpu().float()
    s = v.to(torch.bfloat16).double() / hc
    out = v.double().clone()
    out[:, :act_cols] = (s / (1.0 + torch.exp(-s)))[:, :act_cols]
    return out


def moe_layer(x: torch.Tensor, logits: torch.Tensor, w13: tuple, w2: tuple, topk: int, renorm: bool = True,
              tokens: np.ndarray | None = None, route_out=None, acc_dtype=torch.float32) -> dict:
    """The whole layer on the CPU: route -> per-token fp8 quant -> gate_up -> silu*up + quant -> down (router weight
    folded) -> top-k sum. w13 = (packed [E, 2I, H/2], e8m0 [E, 2I, H/32]) and w2 = (packed [E, H, I/2],
    e8m0 [E, H, I/32]) uint8, in checkpoint layout and indexable by expert. `tokens` restricts the math to those
    tokens (routing and quant are per token, so any subset is exact). Returns every intermediate as numpy."""
    T, H = x.shape
    w, ids = route_out if route_out is not None else route(logits, topk, renorm)
    tok = np.arange(T) if tokens is None else np.asarray(tokens)
    rows = (tok[:, None] * topk + np.arange(topk)[None, :]).reshape(-1)
    xq, xs = quant_rows_fp8(x)
    flat_ids = ids.reshape(-1)
    p13, e13 = w13
    p2, e2 = w2
    deq13 = lambda e: mxfp4_dequant(p13[e], e13[e], torch.float32)
    deq2 = lambda e: mxfp4_dequant(p2[e], e2[e], torch.float32)
    gate_up = grouped_gemm(xq, xs, deq13, flat_ids, topk, None, rows, acc_dtype)          # [R, 2I] bf16 bits
    aq, a_s, _ = silu_mul_quant_fp8(bits_to_bf16(gate_up))
    # down: the A row of routed row rows[i] is aq[i]; the router weight folds into the epilogue
    tw = w.reshape(-1)[rows]
    local = np.arange(rows.size)
    down = grouped_gemm(aq, a_s, deq2, flat_ids[rows], 1, tw, local, acc_dtype)
    out = moe_sum(bits_to_bf16(down.reshape(tok.size, topk, -1)))
    return dict(w=w, ids=ids, xq=xq, xs=xs, rows=rows, gate_up=gate_up, aq=aq, a_s=a_s, down=down, out=out,
                tokens=tok)


class LruState:
    """The device LRU expert cache's state (reference moe/cache.py:193-206): table [E] expert -> slot or -1,
    map_cold [E] expert -> itself when not resident else -1, slot_expert [S], slot_stamp [S] int64, step."""

    def __init__(self, E: int, S: int):
        self.E, self.S = E, S
        self.table = np.full(E, -1, dtype=np.int32)
        self.map_cold = np.arange(E, dtype=np.int32)
        self.slot_expert = np.full(S, -1, dtype=np.int32)
        self.slot_stamp = np.zeros(S, dtype=np.int64)
        self.step = 0

    def copy(self) -> "LruState":
        c = LruState(self.E, self.S)
        c.table, c.map_cold = self.table.copy(), self.map_cold.copy()
        c.slot_expert, c.slot_stamp, c.step = self.slot_expert.copy(), self.slot_stamp.copy(), self.step
        return c


def lru_manage(st: LruState, ids, max_distinct: int, max_inserts: int):
    """One manage call (reference kernels/third_party/davetha/r4d_lru.hip:187-274), in place on `st`. Returns
    (routed flags uint8 [E], miss list [(expert, slot)] in insert order).

    step += 1; routed = the valid ids' experts. More than max_distinct distinct experts: nothing else changes (the
    step reads through; :222). Otherwise resident routed experts get stamp = step (:229-233); the non-resident routed
    ones, in expert-id order, are the misses, at most max_inserts (:236-245); victims are the slots whose expert is
    not routed, taken in ascending (stamp << 20 | slot) order (:108-183), the r-th miss into the r-th victim, as many
    as there are victims; an evicted expert goes cold (table -1, map_cold itself) and the inserted one resident
    (:91-105)."""
    E, S = st.E, st.S
    st.step += 1
    ids = np.asarray(ids, dtype=np.int64).reshape(-1)
    routed = np.zeros(E, dtype=np.uint8)
    v = ids[(ids >= 0) & (ids < E)]
    routed[v] = 1
    if int(routed.sum()) > max_distinct:
        return routed, []
    for e in np.flatnonzero(routed):
        if st.table[e] >= 0:
            st.slot_stamp[st.table[e]] = st.step
    misses = [int(e) for e in np.flatnonzero(routed) if st.table[e] < 0][:max_inserts]
    if not misses:
        return routed, []
    evictable = [i for i in range(S) if not (st.slot_expert[i] >= 0 and routed[st.slot_expert[i]])]
    victims = sorted(evictable, key=lambda i: (int(st.slot_stamp[i]) << 20) | i)[:len(misses)]
    out = []
    for e, sl in zip(misses, victims):
        old = int(st.slot_expert[sl])
        if old >= 0:
            st.table[old] = -1
            st.map_cold[old] = old
        st.slot_expert[sl] = e
        st.slot_stamp[sl] = st.step
        st.table[e] = sl
        st.map_cold[e] = -1
        out.append((e, sl))
    return routed, out


def lru_gather(arena: np.ndarray, store: np.ndarray, misses) -> None:
    """Copy each missed expert's slab from the host store into its slot (reference r4d_lru.hip:276-303)."""
    for e, sl in misses:
        arena[sl] = store[e]
