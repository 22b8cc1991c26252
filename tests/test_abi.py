"""The C-ABI library loads and exports every symbol include/r9k.h declares, and shape errors come back as the
documented return codes before anything touches a GPU (CPU only: no kernel launches)."""
import ctypes
import os
import re

from r9700_vllm.kernels import moe as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "r9k.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"^\s*(?:int|long)\s+(r9k_\w+)\s*\(", src, flags=re.M)


def test_header_symbols_exported():
    names = declared_symbols()
    assert len(names) >= 18, names
    L = ctypes.CDLL(K._lib_path())
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_python_binding_contract():
    L = K.lib()
    assert L.r9k_moe_block() == 16
    assert L.r9k_fold_supported() == 0
    assert L.r9k_moe_route_max_experts() == 1024 and L.r9k_moe_route_max_topk() == 16
    assert K.prefill_block(17) == 64 and L.r9k_moe_prefill_bm(20) == -1 and L.r9k_moe_prefill_bk(-1) == -1


def test_shape_errors_before_launch():
    L = K.lib()
    z = 0
    # N % 16, K % 32, bad MT (the reference's -1 / -2 / -7)
    assert L.r9k_moe_mxfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 17, 2, 4, 2, 1, z) == -1
    assert L.r9k_moe_mxfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 48, 16, 2, 4, 2, 1, z) == -2
    assert L.r9k_moe_mxfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 16, 2, 4, 2, 3, z) == -7
    # the launch shape is read only with MT bit 5 set: a partial or unbuilt shape is -5 (SK = 5 is one of the
    # reference's gfx1201 knob sets, which without the bit are ignored)
    assert K.MT_SHAPE == 32
    assert L.r9k_moe_mxfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 16, 0, 4, 2, 1 | 32, z) == -5
    assert L.r9k_moe_mxfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 640, 16, 2, 5, 2, 1 | 32, z) == -5
    assert L.r9k_moe_4bit_prefill(0, 1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 16, 99, z) == -7
    assert L.r9k_moe_4bit_prefill(3, 1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 16, 17, z) == -8
    # native NVFP4 prefill: 64-row cfg 17 is refused (-7); nothing to do for numel == 0 (no launch)
    assert L.r9k_moe_4bit_prefill(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 16, 17, z) == -7
    assert L.r9k_moe_4bit_prefill(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 0, 1, 64, 16, 2, z) == 0
    # native NVFP4: N % 16, K % 16, K % (16 SK), bad MT; nothing to do for numel == 0 (every case returns before a
    # launch)
    assert L.r9k_moe_nvfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 17, 2, 1, 2, 1, z) == -1
    assert L.r9k_moe_nvfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 72, 16, 2, 1, 2, 1, z) == -2
    assert L.r9k_moe_nvfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 96, 16, 2, 4, 2, 1, z) == -2
    assert L.r9k_moe_nvfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 16, 1, 64, 16, 2, 1, 2, 3, z) == -7
    assert L.r9k_moe_nvfp4a8(1, 1, 1, 1, 1, 1, 1, 1, 1, z, 0, 0, 4, 0, 1, 64, 16, 2, 1, 2, 1, z) == 0
    # route: topk > 16, E > 1024, blk not a power of two (the reference returns 1)
    assert L.r9k_moe_route(1, 64, 1, 1, 1, 1, 1, 1, 1, 64, 17, 1, 16, z) == 1
    assert L.r9k_moe_route(1, 2048, 1, 1, 1, 1, 1, 1, 1, 2048, 8, 1, 16, z) == 1
    assert L.r9k_moe_route(1, 64, 1, 1, 1, 1, 1, 1, 1, 64, 8, 1, 24, z) == 1
    assert L.r9k_moe_topk(1, 64, 1, 1, 1, 64, 65, 1, z) == 1
    assert L.r9k_moe_align(1, 100000, 64, 64, 1, 1, 1, 1, 1, z) == 1          # scratch too small
    assert L.r9k_moe_align_scratch_ints(4096, 64) == 1
    assert L.r9k_moe_align_scratch_ints(65536, 288) == 16 + 32 * 288          # 16 unused ints, 32 chunk histograms
    # sum: N % 8
    assert L.r9k_moe_sum(16, 0, 16, 1, 8, 12, 0, 12, z) == 1
    # quant: nothing to do for M == 0; tiled gate refused
    assert L.r9k_quant_rows_fp8(1, 1, 1, 0, 64, 64, z) == 0
    assert L.r9k_quant_rows_fp8_gate(16, 16, 16, 16, 16, 1, 64, 64, 1, z) == -3
    # router GEMM: M, split, K % (8 split), strides / alignment, act_cols with hc <= 0
    from r9700_vllm import router as R
    Lr = R.lib()
    assert Lr.r9k_router_max_m() == 32
    assert Lr.r9k_router_gemm(16, 64, 16, 64, 16, 64, 33, 64, 64, 1, 1, 0, 1.0, z) == -1
    assert Lr.r9k_router_gemm(16, 64, 16, 64, 16, 64, 1, 64, 4, 1, 1, 0, 1.0, z) == -1
    assert Lr.r9k_router_gemm(16, 64, 16, 64, 16, 64, 1, 64, 64, 3, 1, 0, 1.0, z) == -2
    assert Lr.r9k_router_gemm(16, 64, 16, 64, 16, 64, 1, 64, 72, 2, 1, 0, 1.0, z) == -3
    assert Lr.r9k_router_gemm(16, 60, 16, 64, 16, 64, 1, 64, 64, 1, 1, 0, 1.0, z) == -4
    assert Lr.r9k_router_gemm(24, 64, 16, 64, 16, 64, 1, 64, 64, 1, 1, 0, 1.0, z) == -4
    # device block choice: null table counts, negative sizes (before any launch)
    assert L.r9k_moe_pick_blocks(0, 16, 64, 256, 22, z) == -1
    assert L.r9k_moe_pick_blocks(16, 16, 64, 0, 22, z) == -1
    assert L.r9k_moe_pick_blocks(16, 16, -1, 256, 22, z) == -1
    # expert cache: E / S / mk, the insert cap, pointers, int64 alignment; gather grid, slab sizes and alignment;
    # map ids with nothing to do; host allocation of nothing (all return before a HIP call)
    from r9700_vllm.moe import cache as C
    Lc = C._L()
    p8 = [8] * 8
    assert Lc.r4d_lru_manage(8, 4, 0, 1, 1, 1, *p8, z) == -1
    assert Lc.r4d_lru_manage(8, 4, 8192 + 1, 1, 1, 1, *p8, z) == -1
    assert Lc.r4d_lru_manage(8, 4, 64, 1025, 1, 1, *p8, z) == -1
    assert Lc.r4d_lru_manage(8, 4, 8, 16, 1, 1, *p8, z) == -1                   # more slots than experts
    assert Lc.r4d_lru_manage(8, 4, 64, 16, 1, 17, *p8, z) == -2
    assert Lc.r4d_lru_manage(8, 4, 64, 16, 1, 4, 8, 8, 8, 8, 8, 8, 0, 8, z) == -3
    assert Lc.r4d_lru_manage(8, 4, 64, 16, 1, 4, 8, 8, 8, 12, 8, 8, 8, 8, z) == -4
    slabs = [16, 16, 16] * 6
    assert Lc.r4d_lru_gather(*slabs, 16, 16, 0, 16, z) == -2
    assert Lc.r4d_lru_gather(*slabs, 16, 16, 64, 65536, z) == -2
    assert Lc.r4d_lru_gather(*slabs, 0, 16, 64, 16, z) == -3
    assert Lc.r4d_lru_gather(*([16, 16, 24] + [16, 16, 16] * 5), 16, 16, 64, 16, z) == -4
    assert Lc.r4d_lru_gather(*([16, 24, 16] + [16, 16, 16] * 5), 16, 16, 64, 16, z) == -4
    assert Lc.r4d_lru_gather(*([0, 16, 16] + [16, 16, 16] * 5), 16, 16, 64, 16, z) == -3
    assert Lc.r9k_lru_manage_map(8, 4, 64, 16, 1, 4, *p8, 8, 0, z) == -3          # hot without cold
    assert Lc.r9k_lru_manage_map(8, 4, 64, 16, 1, 17, *p8, 8, 8, z) == -2
    # manage + tables with the folded input quant: rows past 64, a hidden size off the 8-value grid or past 4096, a row
    # stride below H, a row base off 16 bytes (-7); E past one workgroup's tables is not served (2)
    mt = (8, 4, 64, 16, 16, 4, *p8, 16, 8, 8, 8, 0, 0, 0, 8)
    assert Lc.r9k_lru_manage_tables(*mt, 16, 2048, 2048, 65, 16, 16, z) == -7
    assert Lc.r9k_lru_manage_tables(*mt, 16, 2048, 2044, 4, 16, 16, z) == -7
    assert Lc.r9k_lru_manage_tables(*mt, 16, 8192, 8192, 4, 16, 16, z) == -7
    assert Lc.r9k_lru_manage_tables(*mt, 16, 1024, 2048, 4, 16, 16, z) == -7
    assert Lc.r9k_lru_manage_tables(*mt, 8, 2048, 2048, 4, 16, 16, z) == -7
    assert Lc.r9k_lru_manage_tables(8, 4, 2048, 16, 16, 4, *p8, 16, 8, 8, 8, 0, 0, 0, 8, 0, 0, 0, 0, 0, 0, z) == 2
    assert Lc.r9k_lru_map_ids(16, 0, 64, 16, 16, 16, 16, z) == 0
    assert Lc.r9k_lru_map_ids(16, -1, 64, 16, 16, 16, 16, z) == -1
    assert Lc.r9k_lru_map_ids(0, 4, 64, 16, 16, 16, 16, z) == -3
    assert Lc.r9k_host_alloc(0) == 0 and Lc.r9k_host_free(0) == 0
    assert Lr.r9k_router_gemm(16, 64, 16, 64, 16, 64, 1, 64, 64, 1, 1, 8, 0.0, z) == -7
    # converter: K % 32
    assert L.r9k_nvfp4_to_mxfp4(16, 16, 16, 16, 16, 4, 48, z) == -2
    assert L.r9k_quantize_mxfp4_search(16, 16, 16, 4, 40, z) == -2
