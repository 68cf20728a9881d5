"""The C-ABI library (no GPU needed): it loads, exports every entry point declared in
include/matris_hip.h, and its host-side logic (planning, workspace sizing, argument
validation before any launch) behaves as documented."""
import ctypes
import os
import re

import numpy as np
import pytest

from matris_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "matris_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(matris_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmatris_hip.so not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_and_loader_agree():
    assert _declared() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.matris_version().decode().startswith("matris_hip")


def test_radius_graph_plan_host_only(lib):
    grid = (ctypes.c_int * 3)()
    search = (ctypes.c_int * 3)()
    lat = np.ascontiguousarray(np.eye(3) * 78.5)
    assert lib.matris_radius_graph_plan(lat.ctypes.data_as(ctypes.c_void_p), 6.0, grid, search) == 0
    assert list(grid) == [13, 13, 13] and list(search) == [2, 2, 2]
    small = np.ascontiguousarray(np.eye(3) * 3.0)
    assert lib.matris_radius_graph_plan(small.ctypes.data_as(ctypes.c_void_p), 6.0, grid, search) == 0
    assert list(grid) == [1, 1, 1] and list(search) == [4, 4, 4]  # images -4..4 reach 6 A
    flat = np.ascontiguousarray(np.diag([3.0, 3.0, 0.0]))
    assert lib.matris_radius_graph_plan(flat.ctypes.data_as(ctypes.c_void_p), 6.0, grid, search) == -1001


def test_workspace_sizes_are_monotone(lib):
    g = (ctypes.c_int * 3)(4, 4, 4)
    a = lib.matris_radius_graph_workspace_bytes(1000, g)
    b = lib.matris_radius_graph_workspace_bytes(2000, g)
    assert 0 < a < b
    assert lib.matris_pair_edges_workspace_bytes(10) < lib.matris_pair_edges_workspace_bytes(10000)
    assert lib.matris_csr_workspace_bytes(100, 10) < lib.matris_csr_workspace_bytes(100, 100000)


def test_arguments_rejected_before_launch(lib):
    # seg_sum: leading dimension below the 128-wide row, or a column block past ldx
    assert lib.matris_seg_sum(None, 64, 0, ctypes.c_void_p(8), None, 1, 1.0, 0, ctypes.c_void_p(8), None) == -1001
    assert lib.matris_seg_sum(None, 256, 192, ctypes.c_void_p(8), None, 1, 1.0, 0, ctypes.c_void_p(8), None) == -1001
    # gated MLP: 5 sources, or a K that is not a multiple of 128
    src = (ctypes.c_void_p * 4)()
    v16 = ctypes.c_void_p(16)
    assert lib.matris_gmlp_fwd(10, 5, src, None, *([v16] * 6), 1e-7, v16, None, None, None, None, None, 6,
                               None) == -1001
    assert lib.matris_gmlp_bwd(10, 200, *([v16] * 7), 1e-7, v16, None, 0, None, 6, None) == -1001
    # unknown MFMA mode; residual output without its source; accumulate without g_x0
    assert lib.matris_gmlp_bwd(10, 256, *([v16] * 7), 1e-7, v16, None, 0, None, 5, None) == -1001
    src1 = (ctypes.c_void_p * 4)(16)
    assert lib.matris_gmlp_fwd(10, 1, src1, None, *([v16] * 6), 1e-7, v16, None, None, None, v16, v16, 6,
                               None) == -1001
    assert lib.matris_gmlp_bwd(10, 256, *([v16] * 7), 1e-7, v16, None, 1, None, 6, None) == -1001
    # gather after GEMM: 0 or 5 projected blocks; no source at all; 4 projected sources;
    # a projected row stride below 256 or not a multiple of 4; a misaligned projected table
    assert lib.matris_gmlp_project(10, v16, v16, 0, v16, 6, None) == -1001
    assert lib.matris_gmlp_project(10, v16, v16, 5, v16, 6, None) == -1001
    pj = (ctypes.c_void_p * 3)(16, 16, 16)
    ld = (ctypes.c_int64 * 3)(256, 512, 512)
    tail = (v16, v16, v16, v16, v16, 1e-7, v16, None, None, None, None, None, 6, None)
    assert lib.matris_gmlp_fwd_proj(10, 0, None, None, 0, pj, None, ld, None, *tail) == -1001
    assert lib.matris_gmlp_fwd_proj(10, 0, None, None, 4, pj, None, ld, None, *tail) == -1001
    assert lib.matris_gmlp_fwd_proj(10, 0, None, None, 1, pj, None, (ctypes.c_int64 * 3)(128, 0, 0), None,
                                    *tail) == -1001
    assert lib.matris_gmlp_fwd_proj(10, 0, None, None, 1, pj, None, (ctypes.c_int64 * 3)(258, 0, 0), None,
                                    *tail) == -1001
    assert lib.matris_gmlp_fwd_proj(10, 0, None, None, 1, (ctypes.c_void_p * 3)(8), None, ld, None,
                                    *tail) == -1001
    assert lib.matris_gmlp_fwd_proj(10, 1, None, None, 1, pj, None, ld, v16, *tail) == -1001
    # dense layers: misaligned row pointer, null operand, unknown mode, residual without weight
    assert lib.matris_ffn_fwd(10, ctypes.c_void_p(8), v16, v16, v16, None, None, None, 6, None) == -1001
    assert lib.matris_ffn_fwd(10, v16, v16, v16, v16, None, v16, None, 6, None) == -1001
    assert lib.matris_ffn_bwd(10, v16, None, v16, v16, v16, None, None, 6, None) == -1001
    assert lib.matris_pair_fwd(10, v16, v16, v16, v16, 1, None) == -1001
    assert lib.matris_pair_bwd(-1, v16, v16, v16, v16, None, None, 0, 0, None) == -1001
    # attention backward: gradient row stride below 128; envelope aggregation: null operand
    assert lib.matris_attn_bwd(10, 5, v16, v16, 128, None, v16, v16, v16, v16, v16, v16, v16, v16, v16, 64, v16,
                               v16, v16, None, None) == -1001
    assert lib.matris_env_agg_fwd(5, v16, None, v16, None, v16, v16, v16, None) == -1001
    assert lib.matris_env_agg_bwd(10, 5, v16, v16, v16, v16, v16, v16, v16, None, 0, None, v16, None) == -1001
    # weight packing: n not a multiple of 32, k not a multiple of 16, unknown mode
    assert lib.matris_pack_b(48, 16, v16, 6, v16, None) == -1001
    assert lib.matris_pack_b(32, 24, v16, 6, v16, None) == -1001
    assert lib.matris_pack_b(32, 16, v16, 5, v16, None) == -1001
    assert lib.matris_ffn_fwd(10, v16, v16, v16, v16, None, None, None, 1, None) == -1001
    assert lib.matris_pack_b_bytes(256, 384, 6) == 256 * 384 * 6
    assert lib.matris_pack_b_bytes(256, 384, 3) == lib.matris_pack_b_bytes(256, 384, 0) == 256 * 384 * 4
    assert lib.matris_pack_b_bytes(256, 384, 2) == 256 * 384 * 4 + 16
    assert lib.matris_status_take(None, None) == -1001
    # envelope weighting: no multiplier table; a row stride below 128; no output
    assert lib.matris_seg_sum_mul(4, 10, v16, 128, 0, v16, None, None, v16, 1.0, 0, v16, None) == -1001
    assert lib.matris_seg_sum_mul(4, 10, v16, 64, 0, v16, None, v16, v16, 1.0, 0, v16, None) == -1001
    assert lib.matris_gather_mul(10, v16, None, v16, None, 0, None, None) == -1001
    # learnable envelope: K outside 1..8, a misaligned env; projected sums: K = 0, long
    # segments (rows_hint above 4 per segment), no projection output
    assert lib.matris_env_linear(10, 9, v16, v16, v16, None) == -1001
    assert lib.matris_env_linear(10, 0, v16, v16, v16, None) == -1001
    assert lib.matris_env_linear(10, 7, v16, v16, ctypes.c_void_p(8), None) == -1001
    assert lib.matris_env_linear(0, 7, v16, v16, v16, None) == 0
    # narrow segment sums: width outside 1..32
    assert lib.matris_seg_sum_narrow(4, v16, v16, 0, v16, None) == -1001
    assert lib.matris_seg_sum_narrow(4, v16, v16, 33, v16, None) == -1001
    assert lib.matris_seg_sum_narrow(0, None, None, 9, None, None) == 0
    assert lib.matris_seg_sum_mul_proj(4, 8, v16, 128, 0, v16, None, v16, v16, 1.0, v16, 0, 0, v16, None) == -1001
    assert lib.matris_seg_sum_mul_proj(4, 40, v16, 128, 0, v16, None, v16, v16, 1.0, v16, 7, 1, v16, None) == -1001
    assert lib.matris_seg_sum_mul_proj(4, 8, v16, 128, 0, v16, None, v16, v16, 1.0, v16, 7, 0, None, None) == -1001
    assert lib.matris_env_agg_bwd_env_proj(5, v16, v16, v16, v16, v16, v16, None, v16, 9, 0, v16, v16, None) == -1001
    assert lib.matris_env_agg_bwd_env_proj(5, v16, v16, v16, v16, v16, v16, None, None, 7, 1, v16, v16, None) == -1001
    # attention + pair backward: MODE 6 (three planes), a short row stride, res_w without base
    pa = [v16, v16, 128, v16, v16, v16, v16, v16, v16, v16, v16, v16, 256, v16, v16, v16]
    assert lib.matris_attn_pair_bwd(8, *pa, 6, v16, v16, None) == -1001
    assert lib.matris_attn_pair_bwd(8, *pa[:2], 64, *pa[3:], 2, v16, v16, None) == -1001
    assert lib.matris_attn_pair_bwd(8, *pa[:13], None, v16, v16, 2, v16, v16, None) == -1001
    assert lib.matris_attn_pair_bwd(0, *pa, 2, v16, v16, None) == 0
    # positions: a negative count, atoms without a lattice; nothing to do without atoms or strain
    assert lib.matris_frac_to_cart(-1, v16, v16, v16, None, None) == -1001
    assert lib.matris_frac_to_cart(3, v16, None, v16, v16, None) == -1001
    assert lib.matris_frac_to_cart(0, None, None, None, None, None) == 0
    # the batch form: no graphs; atoms without a graph index; nothing to do without atoms or strain
    assert lib.matris_frac_to_cart_batch(3, 0, v16, v16, v16, v16, None, None) == -1001
    assert lib.matris_frac_to_cart_batch(3, 2, v16, v16, None, v16, None, None) == -1001
    assert lib.matris_frac_to_cart_batch(-1, 2, v16, v16, v16, v16, None, None) == -1001
    assert lib.matris_frac_to_cart_batch(0, 2, None, None, None, None, None, None) == 0
    # batched edge geometry: no graphs; edges without a graph index; a strain gradient
    # without a strain; a strain without the graphs' row ranges
    assert lib.matris_edge_geom_fwd_batch(0, 4, *([v16] * 11), None) == -1001
    assert lib.matris_edge_geom_fwd_batch(2, 4, *([v16] * 6), None, *([v16] * 4), None) == -1001
    assert lib.matris_edge_geom_fwd_batch(2, 4, v16, None, *([v16] * 9), None) == -1001
    bw = [v16] * 17
    assert lib.matris_edge_geom_bwd_batch(0, 3, 4, *bw, None) == -1001
    assert lib.matris_edge_geom_bwd_batch(2, 3, 4, *bw[:6], None, *bw[7:], None) == -1001
    assert lib.matris_edge_geom_bwd_batch(2, 3, 4, *bw[:12], None, None, *bw[14:], None) == -1001
    assert lib.matris_csr_build_deferred(10, None, 1, 4, v16, v16, v16, 1, None) == -1001
    # neighbour-list reuse: no atoms; a workspace below its size; a non-positive cutoff
    big = 1 << 20
    assert lib.matris_skin_filter_count(0, 0, v16, v16, 6.0, 1e-8, None, None, None, v16, v16, v16, v16, v16, big,
                                        None) == -1001
    assert lib.matris_skin_filter_count(4, 10, v16, v16, 6.0, 1e-8, v16, v16, v16, v16, v16, v16, v16, v16, 8,
                                        None) == -1001
    assert lib.matris_skin_filter_fill(4, 10, v16, v16, 0.0, 1e-8, v16, v16, v16, v16, v16, v16, v16, v16, v16, big,
                                       None) == -1001
    assert lib.matris_skin_filter_workspace_bytes(1000) > lib.matris_skin_filter_workspace_bytes(10) > 0
    # empty work is a no-op success
    assert lib.matris_seg_sum(None, 128, 0, ctypes.c_void_p(8), None, 0, 1.0, 0, ctypes.c_void_p(8), None) == 0
    assert lib.matris_ffn_fwd(0, v16, v16, v16, v16, None, None, None, 3, None) == 0
    assert lib.matris_env_agg_fwd(0, v16, v16, v16, None, v16, v16, v16, None) == 0
