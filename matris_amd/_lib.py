"""Loader for the C-ABI library libmatris_hip.so (declared in include/matris_hip.h).

The library is built in-tree by `build()` (hipcc, gfx950) and loaded with ctypes.  The
product path has no fallback: if the library is missing, or if no ROCm GPU is visible
when an op runs, the call raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading
from concurrent.futures import ThreadPoolExecutor

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(_HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(_HERE), "include")
LIB_PATH = os.path.join(CSRC, "libmatris_hip.so")
SOURCES = ["graph.hip", "segment.hip", "gmlp.hip", "mlp.hip", "basis.hip", "silu.hip", "readout.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops"]

ERRORS = {
    -1001: "MATRIS_E_ARG (invalid argument)",
    -1002: "MATRIS_E_CAPACITY (capacity exceeded)",
    -1003: "MATRIS_E_IMAGES (periodic image range too large)",
    -1004: "MATRIS_E_UNPAIRED (directed edge without reverse partner)",
    -1005: "MATRIS_E_ORDER (edges not in canonical order)",
    -1006: "MATRIS_E_SCRATCH (the call needs more than the static scratch array)",
}

_lock = threading.Lock()
_lib = None


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link libmatris_hip.so (always rebuilds)."""
    objs = []

    def one(src):
        obj = os.path.join(CSRC, src.replace(".hip", ".o"))
        cmd = [HIPCC, *HIP_FLAGS, "-I", INCLUDE, "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
        if verbose:
            print(" ".join(cmd))
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(one, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    for o in objs:
        os.remove(o)
    return LIB_PATH


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double
_SZ = ctypes.c_size_t

_SIGS = {
    "matris_version": (ctypes.c_char_p, []),
    "matris_radius_graph_plan": (_I, [_P, _D, _P, _P]),
    "matris_radius_graph_workspace_bytes": (_SZ, [_I64, _P]),
    "matris_radius_graph_count": (_I, [_I64, _P, _P, _D, _D, _P, _P, _P, _P, _P, _SZ, _P]),
    "matris_radius_graph_fill": (_I, [_I64, _P, _D, _D, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "matris_skin_filter_workspace_bytes": (_SZ, [_I64]),
    "matris_skin_filter_count": (_I, [_I64, _I64, _P, _P, _D, _D, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "matris_skin_filter_fill": (_I, [_I64, _I64, _P, _P, _D, _D, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "matris_pair_edges_workspace_bytes": (_SZ, [_I64]),
    "matris_pair_edges": (_I, [_I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "matris_line_graph_workspace_bytes": (_SZ, [_I64, _I64]),
    "matris_line_graph_count": (_I, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _D, _P, _P, _P, _SZ, _P]),
    "matris_line_graph_fill": (_I, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _D, _P, _P, _P]),
    "matris_csr_workspace_bytes": (_SZ, [_I64, _I64]),
    "matris_csr_build": (_I, [_I64, _P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "matris_csr_build_deferred": (_I, [_I64, _P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "matris_csr_build_noalloc": (_I, [_I64, _P, _I64, _I64, _P, _P, _P]),
    "matris_seg_sum": (_I, [_P, _I64, _I64, _P, _P, _I64, _F, _I, _P, _P]),
    "matris_seg_sum2": (_I, [_I64, _I64, _P, _I64, _I64, _P, _P, _F, _P, _I64, _I64, _P, _P, _F, _I, _P, _P, _P,
                             _P]),
    "matris_seg_sum2_runs": (_I, [_I64, _I64, _P, _I64, _I64, _P, _I, _F, _P, _I64, _I64, _P, _P, _F, _I, _P, _P]),
    "matris_gather_rows": (_I, [_P, _P, _I64, _F, _I, _P, _P]),
    "matris_seg_sum_mul": (_I, [_I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _F, _I, _P, _P]),
    "matris_seg_sum_mul_proj": (_I, [_I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _F, _P, _I, _I, _P, _P]),
    "matris_gather_mul": (_I, [_I64, _P, _P, _P, _P, _I, _P, _P]),
    "matris_edge_vec_bwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P]),
    "matris_edge_geom_fwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "matris_frac_to_cart": (_I, [_I64, _P, _P, _P, _P, _P]),
    "matris_frac_to_cart_batch": (_I, [_I64, _I64, _P, _P, _P, _P, _P, _P]),
    "matris_edge_geom_bwd": (_I, [_I64, _I64] + [_P] * 17),
    "matris_edge_geom_fwd_batch": (_I, [_I64, _I64] + [_P] * 11 + [_P]),
    "matris_edge_geom_bwd_batch": (_I, [_I64, _I64, _I64] + [_P] * 17 + [_P]),
    "matris_attn_fwd": (_I, [_I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "matris_attn_bwd": (_I, [_I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P,
                             _P]),
    "matris_attn_bwd_bond": (_I, [_I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _F, _P, _P,
                                  _P, _P]),
    "matris_env_agg_fwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P]),
    "matris_env_agg_bwd": (_I, [_I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P]),
    "matris_env_agg_bwd_env": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "matris_env_agg_bwd_env_proj": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P]),
    "matris_env_linear": (_I, [_I64, _I, _P, _P, _P, _P]),
    "matris_seg_sum_narrow": (_I, [_I64, _P, _P, _I, _P, _P]),
    "matris_readout_fwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P]),
    "matris_readout_bwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _I, _P, _P]),
    "matris_gmlp_fwd": (_I, [_I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _I, _P]),
    "matris_gmlp_project": (_I, [_I64, _P, _P, _I, _P, _I, _P]),
    "matris_gmlp_fwd_proj": (_I, [_I64, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P,
                                  _P, _I, _P]),
    "matris_gmlp_fwd_ffn": (_I, [_I64, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P,
                                 _P, _P, _P, _P, _I, _P]),
    "matris_gmlp_fwd_pair": (_I, [_I64, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P,
                                  _P, _P, _P, _P, _I, _P]),
    "matris_gmlp_bwd": (_I, [_I64, _I, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _P, _I, _P]),
    "matris_gmlp_bwd_runs": (_I, [_I64, _I, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _P, _P, _P, _I, _I, _P]),
    "matris_gmlp_bwd_ffn": (_I, [_I64, _I, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _P, _P, _F, _P, _P, _P, _P,
                                 _P, _P, _P, _I, _P]),
    "matris_gmlp_bwd_pair": (_I, [_I64, _I, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I,
                                  _P]),
    "matris_gmlp_tile_rows": (_I, []),
    "matris_silu_bwd": (_I, [_I64, _P, _P, _P, _P]),
    "matris_silu_grad_bwd": (_I, [_I64, _P, _P, _P, _P, _P, _P]),
    "matris_bessel_fwd": (_I, [_I64, _I, _P, _P, _D, _D, _P, _P]),
    "matris_bessel_bwd": (_I, [_I64, _I, _P, _P, _D, _D, _P, _I, _P, _P]),
    "matris_edge_embed_fwd": (_I, [_I64, _P, _P, _P, _D, _P, _D, _I, _D, _P, _P, _P, _P, _D, _P, _P, _P, _P, _P, _P,
                                   _P, _I, _P]),
    "matris_edge_embed_bwd": (_I, [_I64, _P, _P, _P, _D, _P, _D, _I, _D, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _I, _P]),
    "matris_sbf_fwd": (_I, [_I64, _P, _P, _P, _D, _P, _P]),
    "matris_sbf_bwd": (_I, [_I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _D, _I, _P, _P, _P]),
    "matris_pack_b_bytes": (_SZ, [_I64, _I64, _I]),
    "matris_pack_b": (_I, [_I64, _I64, _P, _I, _P, _P]),
    "matris_status_take": (_I, [_P, _P]),
    "matris_ffn_fwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _I, _P]),
    "matris_ffn_bwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _I, _P]),
    "matris_ffn_bwd_env": (_I, [_I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P]),
    "matris_pair_fwd": (_I, [_I64, _P, _P, _P, _P, _I, _P]),
    "matris_pair_bwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "matris_attn_pair_bwd": (_I, [_I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _I, _P, _P,
                                  _P]),
    "matris_tb_embed_fwd": (_I, [_I64, _P, _P, _P, _P, _I, _P]),
    "matris_tb_embed_bwd": (_I, [_I64, _P, _P, _P, _P, _P, _P, _I, _P]),
}

EXPORTED = tuple(_SIGS)


def load():
    """Load the library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc, gfx950) first")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = ERRORS.get(rc, f"hipError_t {rc}")
        raise RuntimeError(f"{what} failed: {msg}")
