"""torch.autograd wrappers over the C-ABI kernels of libmatris_hip.so.

PyTorch supplies device memory, streams and the autograd tape; every op below runs a
hand-written gfx950 kernel and every backward (input gradients only -- forces and
stress never need weight gradients) runs one as well.  There is no CPU fallback: the
ops raise on non-ROCm tensors.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from .. import _lib

D = 128

# MFMA arithmetic of the fused GEMM kernels (include/matris_hip.h MATRIS_MMA_*):
# 0 = fp32 MFMA, 6 = three-way bf16 split (fp32-grade), 2 = fp16 hi/lo split with a
# scaled weight (fp32-grade, half the MFMA work of 6; activations must stay below the
# fp16 range, which the kernels flag), 3 = two-way bf16 split (~2^-16).
MMA_MODES = {"fp32": 0, "f16x3": 2, "bf16x6": 6, "bf16x3": 3}
DEFAULT_MMA = "f16x3"
_MMA = {"mode": MMA_MODES[DEFAULT_MMA]}


def set_mma_precision(name: str) -> None:
    """Select the MFMA arithmetic of the GEMM kernels: one of MMA_MODES (DEFAULT_MMA
    unless set)."""
    _MMA["mode"] = MMA_MODES[name]


def get_mma_precision() -> str:
    return {v: k for k, v in MMA_MODES.items()}[_MMA["mode"]]


class mma_precision:
    """Context manager: run the enclosed ops in another MFMA arithmetic."""

    def __init__(self, name: str):
        self.name, self.prev = name, None

    def __enter__(self):
        self.prev = get_mma_precision()
        set_mma_precision(self.name)
        return self

    def __exit__(self, *exc):
        set_mma_precision(self.prev)


# Bits of the device status word (include/matris_hip.h MATRIS_STATUS_*).
STATUS_F16_RANGE = 1  # an "f16x3" kernel met an activation outside the fp16 range
STATUS_CSR_KEY = 2    # a deferred CSR build met a key outside its segment range


def status_take(device=None) -> int:
    """The device status word (STATUS_* bits) set since the last take; clears it.
    Synchronizes the current stream: one host read per model evaluation."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    bits = ctypes.c_uint(0)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().matris_status_take(ctypes.byref(bits), _stream()), "matris_status_take")
    return int(bits.value)


def f16_range_take(device=None) -> bool:
    """True if an "f16x3" kernel met an activation outside the fp16 range on `device` since
    the last take (its results are unusable).  Clears the whole status word."""
    return bool(status_take(device) & STATUS_F16_RANGE)

# Optional per-launch timing (bench.py): name -> list of (start, end, info) HIP events
# recorded on the launch stream around each kernel call.
_TIMING: dict | None = None
_TIMING_ONLY: frozenset | None = None


def enable_timing(on: bool = True, only=None) -> dict | None:
    """Start (or stop) recording HIP events around the kernel launches of this module: all
    of them, or only the launch names in `only` (fewer events, less host overhead)."""
    global _TIMING, _TIMING_ONLY
    _TIMING = {} if on else None
    _TIMING_ONLY = frozenset(only) if (on and only is not None) else None
    return _TIMING


class _timed:
    __slots__ = ("name", "info", "ev")

    def __init__(self, name, info):
        self.name, self.info, self.ev = name, info, None

    def __enter__(self):
        if _TIMING is not None and (_TIMING_ONLY is None or self.name in _TIMING_ONLY):
            self.ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            self.ev[0].record()

    def __exit__(self, *exc):
        if self.ev is not None:
            self.ev[1].record()
            _TIMING.setdefault(self.name, []).append((self.ev[0], self.ev[1], self.info))


_EXACT_ROWS = [False]


class exact_rows:
    """Context manager: _rows allocates exactly n rows (no view of a larger block) -- for
    outputs handed to torch's dispatcher as custom-op results."""

    def __enter__(self):
        self.prev = _EXACT_ROWS[0]
        _EXACT_ROWS[0] = True
        return self

    def __exit__(self, *exc):
        _EXACT_ROWS[0] = self.prev


def _rows(n: int, cols: int, device, dtype=torch.float32) -> torch.Tensor:
    """An uninitialised [n, cols] tensor whose storage is rounded up to a coarse row count:
    the first n rows of a [cap(n), cols] allocation, cap(n) = n below 2^16 rows, else n
    rounded up to a multiple of 2^(floor(log2 n) - 5) (at most 3% more).  A molecular-
    dynamics run rebuilds its graph every step with slightly different counts; with exact
    sizes the caching allocator's blocks end up a little too small for the next step's
    tensors and, for a large cell, the pool fills with unusable pieces.  Quantised sizes
    let each step reuse the previous step's blocks."""
    if n >= (1 << 16) and not _EXACT_ROWS[0]:
        g = 1 << (n.bit_length() - 6)
        cap = (n + g - 1) // g * g
        return torch.empty(cap, cols, dtype=dtype, device=device)[:n]
    return torch.empty(n, cols, dtype=dtype, device=device)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check_dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("matris_amd ops run on the ROCm device only (no CPU fallback)")


def _f32c(t):
    if t.dtype != torch.float32:
        raise TypeError(f"expected float32, got {t.dtype}")
    return t if t.is_contiguous() else t.contiguous()


def _check_out(t, shape):
    """An output buffer a kernel adds to: fp32, contiguous, on the device, of this shape."""
    if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda or tuple(t.shape) != tuple(shape):
        raise ValueError(f"output buffer must be a contiguous fp32 device tensor of shape {tuple(shape)}")


@dataclass
class Grouping:
    """Rows grouped by an int32 key: rows of segment s are perm[rowptr[s]:rowptr[s+1]]
    (perm None = identity, i.e. rows already sorted by key)."""

    key: torch.Tensor        # int32 [R], segment of each row
    rowptr: torch.Tensor     # int32 [S+1]
    perm: torch.Tensor | None  # int32 [R] or None
    n_seg: int

    @property
    def n_rows(self) -> int:
        return int(self.key.numel())

    @staticmethod
    def build(key: torch.Tensor, n_seg: int, sorted_rows: bool = False, deferred: bool = False) -> "Grouping":
        """Stable CSR of `key` (contiguous int32 device tensor) through matris_csr_build.
        sorted_rows: the caller guarantees key is non-decreasing (perm is the identity).
        deferred: no host read; a key outside [0, n_seg) sets STATUS_CSR_KEY in the
        device status word (status_take) instead of raising here."""
        _check_dev(key)
        if key.dtype != torch.int32 or not key.is_contiguous():
            raise TypeError("Grouping keys must be contiguous int32")
        lib = _lib.load()
        R = key.numel()
        dev = key.device
        rowptr = torch.empty(n_seg + 1, dtype=torch.int32, device=dev)
        # sorted keys: row pointers only (a descent is reported like an out-of-range key)
        perm = None if sorted_rows else _rows(max(R, 1), 1, dev, torch.int32).view(-1)
        ws_bytes = lib.matris_csr_workspace_bytes(R, n_seg)
        ws = _rows(ws_bytes, 1, dev, torch.uint8).view(-1)
        fn = lib.matris_csr_build_deferred if deferred else lib.matris_csr_build
        _lib.check(fn(R, _p(key), 1, n_seg, _p(rowptr), _p(perm), _p(ws), ws_bytes, _stream()), "matris_csr_build")
        return Grouping(key, rowptr, None if sorted_rows else perm[:R], n_seg)


# ------------------------------------------------------------------------------------
# segment sum / gather
# ------------------------------------------------------------------------------------
def seg_sum_narrow_raw(x: torch.Tensor, rowptr: torch.Tensor, n_seg: int) -> torch.Tensor:
    """[n_seg, *x.shape[1:]]: sums of the contiguous row ranges [rowptr[s], rowptr[s+1]) of
    x (at most 32 floats per row) in a fixed order (matris_seg_sum_narrow)."""
    lib = _lib.load()
    x = _f32c(x)
    w = 1
    for d in x.shape[1:]:
        w *= int(d)
    out = torch.empty((n_seg,) + tuple(x.shape[1:]), dtype=torch.float32, device=x.device)
    if rowptr.dtype != torch.int32 or rowptr.numel() != n_seg + 1:
        raise ValueError("seg_sum_narrow_raw: rowptr must be int32 with n_seg + 1 entries")
    with _timed("seg_sum_narrow", dict(rows=x.shape[0], segs=n_seg)):
        _lib.check(lib.matris_seg_sum_narrow(n_seg, _p(rowptr), _p(x), w, _p(out), _stream()),
                   "matris_seg_sum_narrow")
    return out


class SegSumNarrow(torch.autograd.Function):
    """Per-segment sums of narrow rows (seg_sum_narrow_raw) whose backward broadcasts each
    segment's gradient to its rows (segment ids `seg`, int64 [R])."""

    @staticmethod
    def forward(ctx, x, rowptr, seg, n_seg: int):
        ctx.save_for_backward(seg)
        return seg_sum_narrow_raw(x, rowptr, n_seg)

    @staticmethod
    def backward(ctx, g):
        (seg,) = ctx.saved_tensors
        return g.index_select(0, seg), None, None, None


def _seg_src_bytes(grp: "Grouping", rows_read: int | None = None) -> int:
    """Algorithmic bytes of one summed source: its 128-wide rows read once (rows_read of
    them; all of the grouping's rows by default), its int32 permutation and row pointers."""
    r = grp.n_rows if rows_read is None else rows_read
    return 4 * D * r + (4 * grp.n_rows if grp.perm is not None else 0) + 4 * (grp.n_seg + 1)


def seg_sum_raw(x: torch.Tensor, grp: Grouping, scale: float = 1.0, ldx: int = D, col_off: int = 0,
                out: torch.Tensor | None = None, accumulate: bool = False, second=None, base=None,
                tile_rows: int = 0) -> torch.Tensor:
    """out (+)= scale * segment sums of x[:, col_off:col_off+128] over grp; with
    second = (x2, grp2, scale2, ldx2, col_off2) also + scale2 * those of x2 over grp2 (same
    segment count), in the same pass (matris_seg_sum2); with base = (feat [n_seg, 128],
    w [128]) also + w * feat (a residual term).  tile_rows > 0: x holds tile-run partial
    sums of rows ascending by grp's key (gmlp_bwd_raw's runs) and each segment adds one
    partial per tile it spans (matris_seg_sum2_runs; no base)."""
    lib = _lib.load()
    if out is None:
        out = _rows(grp.n_seg, D, x.device)
    rows = grp.n_rows
    if second is not None:
        x2, g2, s2, ld2, off2 = second
        if g2.n_seg != grp.n_seg:
            raise ValueError("seg_sum_raw: both groupings need the same segment count")
        rows = max(rows, g2.n_rows)
        args2 = (_p(x2), ld2, off2, _p(g2.rowptr), _p(g2.perm), s2)
    else:
        args2 = (None, D, 0, None, None, 0.0)
    # algorithmic bytes: each source's rows (a tile-run source: one partial row per tile and
    # segment start), indices and row pointers; out written (and read when accumulated);
    # the base term's rows and weights
    out_b = 4 * D * grp.n_seg * (2 if accumulate else 1)
    b2 = _seg_src_bytes(second[1]) if second is not None else 0
    if tile_rows:
        if grp.perm is not None or base is not None:
            raise ValueError("seg_sum_raw: tile-run partials need rows ascending by segment and no base term")
        nb = _seg_src_bytes(grp, min(grp.n_rows, grp.n_seg + -(-grp.n_rows // int(tile_rows)))) + b2 + out_b
        with _timed("seg_sum", dict(rows=grp.n_rows, segs=grp.n_seg, kind="runs", bytes=nb)):
            _lib.check(lib.matris_seg_sum2_runs(grp.n_seg, rows, _p(x), ldx, col_off, _p(grp.rowptr), int(tile_rows),
                                                scale, *args2, int(accumulate), _p(out), _stream()),
                       "matris_seg_sum2_runs")
        return out
    bx, bw = base if base is not None else (None, None)
    nb = _seg_src_bytes(grp) + b2 + out_b + (4 * D * (grp.n_seg + 1) if base is not None else 0)
    with _timed("seg_sum", dict(rows=grp.n_rows, segs=grp.n_seg, kind="perm" if grp.perm is not None else "sorted",
                                bytes=nb)):
        _lib.check(lib.matris_seg_sum2(grp.n_seg, rows, _p(x), ldx, col_off, _p(grp.rowptr), _p(grp.perm), scale,
                                       *args2, int(accumulate), _p(bx), _p(bw), _p(out), _stream()),
                   "matris_seg_sum2")
    return out


def gather_raw(src: torch.Tensor, idx: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    lib = _lib.load()
    out = _rows(idx.numel(), D, src.device)
    _lib.check(lib.matris_gather_rows(_p(src), _p(idx), idx.numel(), scale, 0, _p(out), _stream()),
               "matris_gather_rows")
    return out


def seg_sum_mul_raw(x: torch.Tensor, grp: Grouping, mul: torch.Tensor, mul_idx: torch.Tensor,
                    out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """out (+)= segment sums over grp of x[r] * mul[mul_idx[r]] (matris_seg_sum_mul)."""
    lib = _lib.load()
    if out is None:
        out = _rows(grp.n_seg, D, x.device)
    nb = _seg_src_bytes(grp) + 4 * D * mul.shape[0] + 4 * grp.n_rows + 4 * D * grp.n_seg * (2 if accumulate else 1)
    with _timed("seg_sum", dict(rows=grp.n_rows, segs=grp.n_seg, kind="mul", bytes=nb)):
        _lib.check(lib.matris_seg_sum_mul(grp.n_seg, grp.n_rows, _p(x), D, 0, _p(grp.rowptr), _p(grp.perm), _p(mul),
                                          _p(mul_idx), 1.0, int(accumulate), _p(out), _stream()),
                   "matris_seg_sum_mul")
    return out


def seg_sum_mul_proj_raw(x: torch.Tensor, grp: Grouping, mul: torch.Tensor, mul_idx: torch.Tensor,
                         proj_wt: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """[n_seg, K]: the segment sums of seg_sum_mul_raw(x, grp, mul, mul_idx) times W, with
    proj_wt = W^T [K, 128] (matris_seg_sum_mul_proj; short segments: at most 4 rows per
    segment on average, e.g. the two directed copies of each bond).  Added to `out` when
    it is given (fp32 contiguous [n_seg, K])."""
    lib = _lib.load()
    wt = _f32c(proj_wt)
    acc = out is not None
    if acc:
        _check_out(out, (grp.n_seg, wt.shape[0]))
    else:
        out = torch.empty(grp.n_seg, wt.shape[0], dtype=torch.float32, device=x.device)
    nb = (_seg_src_bytes(grp) + 4 * D * mul.shape[0] + 4 * grp.n_rows
          + (2 if acc else 1) * 4 * wt.shape[0] * grp.n_seg)
    with _timed("seg_sum", dict(rows=grp.n_rows, segs=grp.n_seg, kind="mul_proj", bytes=nb)):
        _lib.check(lib.matris_seg_sum_mul_proj(grp.n_seg, grp.n_rows, _p(x), D, 0, _p(grp.rowptr), _p(grp.perm),
                                               _p(mul), _p(mul_idx), 1.0, _p(wt), wt.shape[0], int(acc), _p(out),
                                               _stream()),
                   "matris_seg_sum_mul_proj")
    return out


def gather_mul_raw(a: torch.Tensor, ia, b: torch.Tensor, ib, out: torch.Tensor, accumulate: bool = False):
    """out[r] (+)= a[ia[r]] * b[ib[r]] (matris_gather_mul; an index None is the identity)."""
    if out.shape[0] == 0:
        return out
    lib = _lib.load()
    with _timed("gather", (out.shape[0],)):
        _lib.check(lib.matris_gather_mul(out.shape[0], _p(a), _p(ia), _p(b), _p(ib), int(accumulate), _p(out),
                                         _stream()), "matris_gather_mul")
    return out


class _EdgeVec(torch.autograd.Function):
    """vec = cart[tgt] - (cart[src] + shift) with a deterministic CSR backward for cart."""

    @staticmethod
    def forward(ctx, cart, shift, tgt: "Grouping", src: "Grouping"):
        _check_dev(cart, shift)
        ctx.tgt, ctx.src, ctx.n = tgt, src, cart.shape[0]
        return cart.index_select(0, tgt.key) - (cart.index_select(0, src.key) + shift)

    @staticmethod
    def backward(ctx, g):
        g = g.float().contiguous()
        lib = _lib.load()
        g_cart = torch.empty(ctx.n, 3, dtype=torch.float32, device=g.device)
        t, s = ctx.tgt, ctx.src
        with _timed("edge_vec_bwd", (ctx.n,)):
            _lib.check(lib.matris_edge_vec_bwd(ctx.n, _p(g), _p(t.rowptr), _p(t.perm), _p(s.rowptr), _p(s.perm),
                                               _p(g_cart), _stream()), "matris_edge_vec_bwd")
        return g_cart, -g, None, None


def edge_vectors(cart, shift, tgt: "Grouping", src: "Grouping"):
    """cart[tgt] - (cart[src] + shift) (processgraph.py:192-199) for fp32 cart [N,3] and
    shift [E,3]; tgt / src are the atom graph's CSR groupings."""
    return _EdgeVec.apply(cart, shift, tgt, src)


GEOM_PARTS = 512  # MATRIS_GEOM_PARTS: blocks of matris_edge_geom_bwd's per-edge pass


class _EdgeGeometry(torch.autograd.Function):
    """One graph's edge geometry with the strain trick (processgraph.py:169-199) through
    matris_edge_geom_fwd / matris_edge_geom_bwd.  Differentiable in cart and strain; the
    strained lattice and the volume are returned as plain values."""

    @staticmethod
    def forward(ctx, cart, strain, lattice, image, tgt: "Grouping", src: "Grouping"):
        _check_dev(cart, strain, lattice, image)
        cart, lattice, image = _f32c(cart), _f32c(lattice), _f32c(image)
        strain = None if strain is None else _f32c(strain)
        if cart.dim() != 2 or cart.shape[1] != 3 or lattice.numel() != 9 or image.dim() != 2 or \
                image.shape[1] != 3 or (strain is not None and strain.numel() != 9) or \
                tgt.n_rows != image.shape[0] or src.n_rows != image.shape[0] or tgt.n_seg != cart.shape[0] or \
                src.n_seg != cart.shape[0]:
            raise ValueError("edge_geometry: expected cart [N,3], lattice [3,3], strain [1,3,3], image [E,3] and "
                             "groupings of E rows over N atoms")
        E, dev = image.shape[0], cart.device
        length = _rows(E, 1, dev).view(-1)
        unit = _rows(E, 3, dev)
        lat_out = torch.empty(3, 3, device=dev)
        vol = torch.empty(1, 1, 1, device=dev)
        with _timed("edge_geom_fwd", (E,)):
            _lib.check(_lib.load().matris_edge_geom_fwd(E, _p(cart), _p(lattice), _p(strain), _p(image), _p(tgt.key),
                                                        _p(src.key), _p(length), _p(unit), _p(lat_out), _p(vol),
                                                        _stream()), "matris_edge_geom_fwd")
        ctx.save_for_backward(length, unit, cart, strain, lattice, image)
        ctx.tgt, ctx.src = tgt, src
        ctx.mark_non_differentiable(lat_out, vol)
        ctx.set_materialize_grads(False)
        return length, unit, lat_out, vol

    @staticmethod
    def backward(ctx, g_len, g_unit, _g_lat, _g_vol):
        length, unit, cart, strain, lattice, image = ctx.saved_tensors
        N, E, dev = cart.shape[0], image.shape[0], cart.device
        g_len = None if g_len is None else _f32c(g_len)
        g_unit = None if g_unit is None else _f32c(g_unit)
        g_vec = _rows(E, 3, dev)
        partial = torch.empty(9 * GEOM_PARTS, device=dev)
        g_cart = torch.empty(N, 3, device=dev)
        g_strain = torch.empty_like(strain) if (strain is not None and ctx.needs_input_grad[1]) else None
        t, s = ctx.tgt, ctx.src
        with _timed("edge_geom_bwd", (E,)):
            _lib.check(_lib.load().matris_edge_geom_bwd(N, E, _p(g_len), _p(g_unit), _p(length), _p(unit), _p(cart),
                                                        _p(lattice), _p(strain), _p(image), _p(t.rowptr),
                                                        _p(t.perm), _p(s.rowptr), _p(s.perm), _p(g_vec),
                                                        _p(partial), _p(g_cart), _p(g_strain), _stream()),
                       "matris_edge_geom_bwd")
        return g_cart, g_strain, None, None, None, None


class _EdgeGeometryBatch(torch.autograd.Function):
    """A disjoint batch's edge geometry with the strain trick (processgraph.py:169-199,
    each edge with its own graph's lattice and strain) through matris_edge_geom_fwd_batch /
    matris_edge_geom_bwd_batch.  Differentiable in cart and strain; the strained lattices
    and the volumes are returned as plain values."""

    @staticmethod
    def forward(ctx, cart, strain, lattice, image, tgt: "Grouping", src: "Grouping", graph_of_edge, atom_ptr,
                edge_ptr):
        _check_dev(cart, strain, lattice, image, graph_of_edge, atom_ptr, edge_ptr)
        cart, lattice, image = _f32c(cart), _f32c(lattice), _f32c(image)
        strain = None if strain is None else _f32c(strain)
        G = lattice.shape[0]
        E = image.shape[0]
        if cart.dim() != 2 or cart.shape[1] != 3 or lattice.dim() != 3 or tuple(lattice.shape[1:]) != (3, 3) or \
                image.dim() != 2 or image.shape[1] != 3 or (strain is not None and tuple(strain.shape) != (G, 3, 3)) \
                or tgt.n_rows != E or src.n_rows != E or tgt.n_seg != cart.shape[0] or src.n_seg != cart.shape[0] \
                or graph_of_edge.dtype != torch.int32 or tuple(graph_of_edge.shape) != (E,) or \
                tuple(atom_ptr.shape) != (G + 1,) or tuple(edge_ptr.shape) != (G + 1,) or G < 1:
            raise ValueError("edge_geometry_batch: expected cart [N,3], lattice and strain [G,3,3], image [E,3], "
                             "groupings of E rows over N atoms, int32 graph_of_edge [E] and row pointers [G+1]")
        dev = cart.device
        length = _rows(E, 1, dev).view(-1)
        unit = _rows(E, 3, dev)
        lat_out = torch.empty(G, 3, 3, device=dev)
        vol = torch.empty(G, 1, 1, device=dev)
        with _timed("edge_geom_fwd", (E,)):
            _lib.check(_lib.load().matris_edge_geom_fwd_batch(G, E, _p(cart), _p(lattice), _p(strain), _p(image),
                                                              _p(tgt.key), _p(src.key), _p(graph_of_edge),
                                                              _p(length), _p(unit), _p(lat_out), _p(vol), _stream()),
                       "matris_edge_geom_fwd_batch")
        ctx.save_for_backward(length, unit, cart, strain, lattice, image, atom_ptr, edge_ptr)
        ctx.tgt, ctx.src = tgt, src
        ctx.mark_non_differentiable(lat_out, vol)
        ctx.set_materialize_grads(False)
        return length, unit, lat_out, vol

    @staticmethod
    def backward(ctx, g_len, g_unit, _g_lat, _g_vol):
        length, unit, cart, strain, lattice, image, atom_ptr, edge_ptr = ctx.saved_tensors
        G, N, E, dev = lattice.shape[0], cart.shape[0], image.shape[0], cart.device
        g_len = None if g_len is None else _f32c(g_len)
        g_unit = None if g_unit is None else _f32c(g_unit)
        g_vec = _rows(E, 3, dev)
        g_cart = torch.empty(N, 3, device=dev)
        g_strain = torch.empty_like(strain) if (strain is not None and ctx.needs_input_grad[1]) else None
        t, s = ctx.tgt, ctx.src
        with _timed("edge_geom_bwd", (E,)):
            _lib.check(_lib.load().matris_edge_geom_bwd_batch(G, N, E, _p(g_len), _p(g_unit), _p(length), _p(unit),
                                                              _p(cart), _p(lattice), _p(strain), _p(image),
                                                              _p(t.rowptr), _p(t.perm), _p(s.rowptr), _p(s.perm),
                                                              _p(atom_ptr), _p(edge_ptr), _p(g_vec), _p(g_cart),
                                                              _p(g_strain), _stream()), "matris_edge_geom_bwd_batch")
        return g_cart, g_strain, None, None, None, None, None, None, None


def edge_geometry_batch(cart, strain, lattice, image, tgt: "Grouping", src: "Grouping", graph_of_edge, atom_ptr,
                        edge_ptr):
    """(length [E], unit [E,3], strained lattices [G,3,3], volumes [G,1,1]) of a disjoint
    batch (processgraph.py:169-199 per graph): cart [N,3], strain [G,3,3] or None, lattice
    [G,3,3], image [E,3] fp32; tgt / src the batch's atom-graph groupings; graph_of_edge int32
    [E]; atom_ptr / edge_ptr int32 [G+1], each graph's contiguous atom and edge rows."""
    return _EdgeGeometryBatch.apply(cart, strain, lattice, image, tgt, src, graph_of_edge, atom_ptr, edge_ptr)


def frac_to_cart(frac: torch.Tensor, lattice: torch.Tensor, with_strain: bool):
    """(cart [N, 3] = frac @ lattice, zero strain [1, 3, 3] or None) of one graph in one
    launch (matris_frac_to_cart; processgraph.py:87 and :173-177), both new tensors without
    autograd history: the caller makes them the leaves forces and stress differentiate."""
    _check_dev(frac, lattice)
    frac, lattice = _f32c(frac), _f32c(lattice)
    if frac.dim() != 2 or frac.shape[1] != 3 or tuple(lattice.shape) != (3, 3):
        raise ValueError("frac_to_cart: frac must be [N, 3] and lattice [3, 3]")
    lib = _lib.load()
    cart = torch.empty_like(frac)
    strain = torch.empty((1, 3, 3), dtype=torch.float32, device=frac.device) if with_strain else None
    _lib.check(lib.matris_frac_to_cart(frac.shape[0], _p(frac), _p(lattice), _p(cart), _p(strain), _stream()),
               "matris_frac_to_cart")
    return cart, strain


def frac_to_cart_batch(frac: torch.Tensor, lattice: torch.Tensor, graph_of_atom: torch.Tensor, with_strain: bool):
    """(cart [N, 3], zero strains [G, 3, 3] or None) of a disjoint batch in one launch
    (matris_frac_to_cart_batch): cart[i] = frac[i] @ lattice[graph_of_atom[i]] with frac
    [N, 3], lattice [G, 3, 3] and graph_of_atom [N] int32, the arithmetic of frac_to_cart
    (processgraph.py:87 per graph).  New tensors without autograd history.  A graph index
    outside [0, G) surfaces in the status word (STATUS_CSR_KEY)."""
    _check_dev(frac, lattice, graph_of_atom)
    frac, lattice = _f32c(frac), _f32c(lattice)
    G = lattice.shape[0]
    if frac.dim() != 2 or frac.shape[1] != 3 or lattice.dim() != 3 or tuple(lattice.shape[1:]) != (3, 3) or G < 1:
        raise ValueError("frac_to_cart_batch: frac must be [N, 3] and lattice [G, 3, 3] with G >= 1")
    if graph_of_atom.dtype != torch.int32 or tuple(graph_of_atom.shape) != (frac.shape[0],):
        raise ValueError("frac_to_cart_batch: graph_of_atom must be int32 [N]")
    graph_of_atom = graph_of_atom.contiguous()
    lib = _lib.load()
    cart = torch.empty_like(frac)
    strain = torch.empty((G, 3, 3), dtype=torch.float32, device=frac.device) if with_strain else None
    _lib.check(lib.matris_frac_to_cart_batch(frac.shape[0], G, _p(frac), _p(lattice), _p(graph_of_atom), _p(cart),
                                             _p(strain), _stream()), "matris_frac_to_cart_batch")
    return cart, strain


def edge_geometry(cart, strain, lattice, image, tgt: "Grouping", src: "Grouping"):
    """(length [E], unit [E,3], strained lattice [3,3], volume [1,1,1]) of one graph:
    processgraph.py:169-199 with sym = (strain + strain^T)/2 applied to the positions and
    the lattice (strain [1,3,3] or None), vec = x'[tgt] - (x'[src] + image L').  cart [N,3],
    lattice [3,3] and image [E,3] contiguous fp32; tgt / src the atom graph's groupings."""
    return _EdgeGeometry.apply(cart, strain, lattice, image, tgt, src)


class _SegSum(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, grp: Grouping, scale: float):
        _check_dev(x)
        x = _f32c(x)
        ctx.grp, ctx.scale = grp, scale
        return seg_sum_raw(x, grp, scale)

    @staticmethod
    def backward(ctx, g):
        g = _f32c(g)
        return gather_raw(g, ctx.grp.key, ctx.scale), None, None


class _Gather(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, grp: Grouping):
        _check_dev(src)
        src = _f32c(src)
        ctx.grp = grp
        return gather_raw(src, grp.key)

    @staticmethod
    def backward(ctx, g):
        g = _f32c(g)
        return seg_sum_raw(g, ctx.grp), None


def seg_sum(x, grp: Grouping, scale: float = 1.0):
    """out[s] = scale * sum of x rows with key s (aggregate(), functions.py:129-160).
    Rows of another width than 128 (feature widths other than MatRIS-10M's) are summed by
    torch on the device."""
    if x.dim() != 2 or x.shape[1] != D:
        _check_dev(x)
        out = torch.zeros(grp.n_seg, *x.shape[1:], dtype=x.dtype, device=x.device)
        return out.index_add(0, grp.key.long(), x) * scale
    return _SegSum.apply(x, grp, scale)


def gather(src, grp: Grouping):
    """src[grp.key] (torch.index_select), with a deterministic CSR backward (rows of
    another width than 128: torch.index_select itself)."""
    if src.dim() != 2 or src.shape[1] != D:
        _check_dev(src)
        return torch.index_select(src, 0, grp.key.long())
    return _Gather.apply(src, grp)


# ------------------------------------------------------------------------------------
# segment attention
# ------------------------------------------------------------------------------------
def attn_fwd_raw(alpha_t, alpha_s, e, tgt: Grouping, src: Grouping, alpha_grp: Grouping | None):
    """(y_t, y_s, lse_t, lse_s) of matris_attn_fwd."""
    lib = _lib.load()
    R, S = e.shape[0], tgt.n_seg
    dev = e.device
    y_t, y_s = _rows(S, D, dev), _rows(S, D, dev)
    lse_t, lse_s = _rows(S, D, dev), _rows(S, D, dev)
    aidx = alpha_grp.key if alpha_grp is not None else None
    # algorithmic bytes (in: alpha_t, alpha_s (whole tables when gathered), e; out: y_t, y_s;
    # int32 permutation / alpha index and two row-pointer arrays); lse_t / lse_s are saved
    # statistics, counted apart
    n_alpha = alpha_t.shape[0]
    nb = 4 * D * (2 * n_alpha + R + 2 * S) + (4 * R if src.perm is not None else 0) + \
        (4 * R if aidx is not None else 0) + 8 * (S + 1)
    with _timed("attn_fwd_atom" if aidx is not None else "attn_fwd_line",
                dict(rows=R, segs=S, bytes=nb, saved_bytes=2 * 4 * D * S)):
        _lib.check(lib.matris_attn_fwd(R, S, _p(alpha_t), _p(alpha_s), D, _p(aidx), _p(e), _p(tgt.rowptr),
                                       _p(tgt.perm), _p(src.rowptr), _p(src.perm), _p(y_t), _p(y_s), _p(lse_t),
                                       _p(lse_s), _stream()), "matris_attn_fwd")
    return y_t, y_s, lse_t, lse_s


def attn_bwd_raw(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, tgt: Grouping, src: Grouping,
                 alpha_grp: Grouping | None, ldgy: int = D, g_e_base=None):
    """(g_alpha_t, g_alpha_s, g_e) per row of matris_attn_bwd; g_yt / g_ys may be views
    of row stride ldgy; g_e = g_e_base + attention term when g_e_base is given."""
    lib = _lib.load()
    R, S = e.shape[0], tgt.n_seg
    dev = e.device
    g_at, g_as, g_e = (_rows(R, D, dev) for _ in range(3))
    ag = alpha_grp
    # algorithmic bytes (in: alpha_t, alpha_s, e [R], g_yt, g_ys [S], the fused base term
    # [R]; out: g_alpha_t, g_alpha_s, g_e [R]; target and source keys); y_t, y_s, lse_t,
    # lse_s are saved statistics, counted apart
    nb = 4 * D * (6 * R + 2 * S) + (4 * D * R if g_e_base is not None else 0) + 8 * R + \
        (4 * R if ag is not None else 0)
    with _timed("attn_bwd_atom" if ag is not None else "attn_bwd_line",
                dict(rows=R, segs=S, bytes=nb, saved_bytes=4 * 4 * D * S)):
        _lib.check(lib.matris_attn_bwd(R, S, _p(alpha_t), _p(alpha_s), D, _p(ag.key if ag is not None else None),
                                       _p(e), _p(tgt.key), _p(src.key), _p(y_t), _p(y_s), _p(lse_t), _p(lse_s),
                                       _p(g_yt), _p(g_ys), ldgy, _p(g_at), _p(g_as), _p(g_e), _p(g_e_base),
                                       _stream()), "matris_attn_bwd")
    return g_at, g_as, g_e


def attn_pair_bwd_raw(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_y, tgt: Grouping, src: Grouping, base,
                      pair: "_WeightPack", res_w, mode: int):
    """(g_e, g_tb) of matris_attn_pair_bwd on the line graph: g_e = base + attention term (as
    attn_bwd_raw), g_tb = g_as W_s + g_at W_t + res_w * base (as pair_bwd_raw of attn_bwd_raw's
    logit gradients, which are not materialised).  g_y = [g_yt | g_ys] rows of 256; modes
    0, 2, 3."""
    lib = _lib.load()
    R, S = e.shape[0], tgt.n_seg
    dev = e.device
    g_e, g_tb = _rows(R, D, dev), _rows(R, D, dev)
    if g_y.shape[1] != 2 * D or g_y.stride(0) != 2 * D:
        raise ValueError("attn_pair_bwd_raw: g_y must be [S, 256] rows")
    # in: alpha_t, alpha_s, e, base [R], g_y [S, 256]; out: g_e, g_tb [R]; keys; the saved
    # statistics y_t, y_s, lse_t, lse_s counted apart
    nb = 4 * D * (4 * R + 2 * S) + 4 * D * 2 * R + 8 * R
    with _timed("attn_bwd_line", dict(rows=R, segs=S, bytes=nb, saved_bytes=4 * 4 * D * S, kind="pair")):
        _lib.check(lib.matris_attn_pair_bwd(R, _p(alpha_t), _p(alpha_s), D, _p(e), _p(tgt.key), _p(src.key), _p(y_t),
                                            _p(y_s), _p(lse_t), _p(lse_s), _p(g_y), _p(g_y[:, D:]), 2 * D, _p(base),
                                            _p(pair.b("cat_t", mode)), _p(res_w), mode, _p(g_e), _p(g_tb),
                                            _stream()), "matris_attn_pair_bwd")
    return g_e, g_tb


def attn_bwd_bond_raw(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, tgt: Grouping, src: Grouping,
                      d2u: Grouping, ldgy: int = D, g_base=None, base_scale: float = 1.0):
    """(g_alpha_t, g_alpha_s) per bond and g_e per directed row of matris_attn_bwd_bond: the
    atom-graph backward with the logits per bond (rows of d2u's segments)."""
    lib = _lib.load()
    R, U = e.shape[0], d2u.n_seg
    dev = e.device
    if alpha_t.shape[0] != U or tgt.key.numel() != R or src.key.numel() != R:
        raise ValueError("attn_bwd_bond_raw: logits per bond, one target / source per directed row")
    g_at, g_as, g_e = _rows(U, D, dev), _rows(U, D, dev), _rows(R, D, dev)
    with _timed("attn_bwd_atom", dict(rows=R, segs=tgt.n_seg)):
        _lib.check(lib.matris_attn_bwd_bond(U, _p(alpha_t), _p(alpha_s), D, _p(e), _p(d2u.rowptr), _p(d2u.perm),
                                            _p(tgt.key), _p(src.key), _p(y_t), _p(y_s), _p(lse_t), _p(lse_s),
                                            _p(g_yt), _p(g_ys), ldgy, _p(g_base), float(base_scale), _p(g_at),
                                            _p(g_as), _p(g_e), _stream()), "matris_attn_bwd_bond")
    return g_at, g_as, g_e


class _SegAttn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, alpha_t, alpha_s, e, tgt: Grouping, src: Grouping, alpha_grp):
        _check_dev(alpha_t, alpha_s, e)
        alpha_t, alpha_s, e = _f32c(alpha_t), _f32c(alpha_s), _f32c(e)
        y_t, y_s, lse_t, lse_s = attn_fwd_raw(alpha_t, alpha_s, e, tgt, src, alpha_grp)
        ctx.save_for_backward(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s)
        ctx.tgt, ctx.src, ctx.alpha_grp = tgt, src, alpha_grp
        return y_t, y_s

    @staticmethod
    def backward(ctx, g_yt, g_ys):
        alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s = ctx.saved_tensors
        g_yt = torch.zeros_like(y_t) if g_yt is None else _f32c(g_yt)
        g_ys = torch.zeros_like(y_s) if g_ys is None else _f32c(g_ys)
        ag = ctx.alpha_grp
        g_at, g_as, g_e = attn_bwd_raw(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, ctx.tgt, ctx.src, ag)
        if ag is not None:  # alpha rows were read through alpha_grp.key: reduce back
            g_at = seg_sum_raw(g_at, ag)
            g_as = seg_sum_raw(g_as, ag)
        return g_at, g_as, g_e, None, None, None


def _dimwise_softmax_torch(a, grp: Grouping):
    """Dimwise_softmax (functions.py:97-127) by torch on the device: per column, exp of the
    row minus its segment's maximum over the segment's sum."""
    key = grp.key.long()
    mx = torch.full((grp.n_seg, a.shape[1]), float("-inf"), dtype=a.dtype, device=a.device).scatter_reduce(
        0, key[:, None].expand_as(a), a, "amax", include_self=False)
    ex = torch.exp(a - mx[key])
    den = torch.zeros(grp.n_seg, a.shape[1], dtype=a.dtype, device=a.device).index_add(0, key, ex)
    return ex / den[key]


def seg_attention(alpha_t, alpha_s, e, tgt: Grouping, src: Grouping, alpha_grp: Grouping | None = None):
    """(y_t, y_s): Dimwise_softmax of alpha by target / source segment times e, summed
    per segment (interaction_block.py:113-134).  Features of another width than 128: the
    same by torch on the device."""
    if e.dim() != 2 or e.shape[1] != D or alpha_t.shape[1] != D:
        _check_dev(alpha_t, alpha_s, e)
        if alpha_grp is not None:
            alpha_t, alpha_s = gather(alpha_t, alpha_grp), gather(alpha_s, alpha_grp)
        y_t = seg_sum(_dimwise_softmax_torch(alpha_t, tgt) * e, tgt)
        y_s = seg_sum(_dimwise_softmax_torch(alpha_s, src) * e, src)
        return y_t, y_s
    return _SegAttn.apply(alpha_t, alpha_s, e, tgt, src, alpha_grp)


# ------------------------------------------------------------------------------------
# envelope-weighted aggregation (line-graph Refinement)
# ------------------------------------------------------------------------------------
def env_agg_fwd_raw(h, env, tgt: Grouping, src: Grouping):
    """(agg, S): agg[b] = env[b] * S[b], S[b] = sum over rows a with target b of
    h[a] * env[source(a)]  (interaction_block.py:243-258)."""
    lib = _lib.load()
    E = env.shape[0]
    agg, S = _rows(E, D, h.device), _rows(E, D, h.device)
    A = h.shape[0]
    with _timed("env_agg_fwd", dict(rows=A, segs=E, bytes=4 * D * (A + 2 * E) + 4 * A + 4 * (E + 1),
                                    saved_bytes=4 * D * E)):
        _lib.check(lib.matris_env_agg_fwd(E, _p(h), _p(env), _p(tgt.rowptr), _p(tgt.perm), _p(src.key), _p(S),
                                          _p(agg), _stream()), "matris_env_agg_fwd")
    return agg, S


def env_agg_bwd_env_raw(h, env, g_agg, S, tgt: Grouping, src: Grouping, proj_wt=None, g_basis=None):
    """(g_env, g_agg_env) of matris_env_agg_bwd_env: g_env as env_agg_bwd_raw returns it and
    g_agg_env = g_agg * env, the per-bond factor ffn_bwd_raw(..., env_term=...) takes.  With
    proj_wt (the envelope's Linear(K, 128) weight transposed, [K, 128]) the first result is
    g_env W [E, K], the gradient of the envelope's basis (matris_env_agg_bwd_env_proj),
    added to g_basis when that is given."""
    lib = _lib.load()
    E = env.shape[0]
    ge = _rows(E, D, h.device)
    if proj_wt is not None:
        wt = _f32c(proj_wt)
        acc = g_basis is not None
        if acc:
            _check_out(g_basis, (E, wt.shape[0]))
        else:
            g_basis = torch.empty(E, wt.shape[0], dtype=torch.float32, device=h.device)
        A = h.shape[0]
        # in: h [A], env, g_agg, S [E] (S saved), target keys, source permutation and pointers;
        # out: g_basis [E, K] (read too when accumulating), g_agg * env [E]
        nb = 4 * D * (A + 3 * E) + 4 * D * E + (2 if acc else 1) * 4 * wt.shape[0] * E + 8 * A + 4 * (E + 1)
        with _timed("env_agg_bwd", dict(rows=A, segs=E, bytes=nb, saved_bytes=4 * D * E)):
            _lib.check(lib.matris_env_agg_bwd_env_proj(E, _p(h), _p(env), _p(g_agg), _p(S), _p(tgt.key),
                                                       _p(src.rowptr), _p(src.perm), _p(wt), wt.shape[0], int(acc),
                                                       _p(g_basis), _p(ge), _stream()), "matris_env_agg_bwd_env_proj")
        return g_basis, ge
    g_env = _rows(E, D, h.device)
    A = h.shape[0]
    nb = 4 * D * (A + 3 * E) + 2 * 4 * D * E + 8 * A + 4 * (E + 1)
    with _timed("env_agg_bwd", dict(rows=A, segs=E, bytes=nb, saved_bytes=4 * D * E)):
        _lib.check(lib.matris_env_agg_bwd_env(E, _p(h), _p(env), _p(g_agg), _p(S), _p(tgt.key), _p(src.rowptr),
                                              _p(src.perm), _p(g_env), _p(ge), _stream()), "matris_env_agg_bwd_env")
    return g_env, ge


def env_linear_raw(basis, wt):
    """The learnable envelope env = basis W^T (matris_env_linear; interaction_block.py:240-246,
    nn.Linear(K, 128, bias=False)): basis [E, K], wt = W^T [K, 128] -> env [E, 128]."""
    lib = _lib.load()
    basis, wt = _f32c(basis), _f32c(wt)
    E, K = basis.shape
    if tuple(wt.shape) != (K, D):
        raise ValueError(f"env_linear_raw: the transposed weight must be [{K}, {D}], got {tuple(wt.shape)}")
    env = _rows(E, D, basis.device)
    with _timed("env_linear", (E,)):
        _lib.check(lib.matris_env_linear(E, K, _p(basis), _p(wt), _p(env), _stream()), "matris_env_linear")
    return env


def env_agg_bwd_raw(h, env, g_agg, S, tgt: Grouping, src: Grouping, g_h, accumulate: bool):
    """g_h (+)= g_agg[tgt] * env[tgt] * env[src]; returns g_env."""
    lib = _lib.load()
    E = env.shape[0]
    g_env = _rows(E, D, h.device)
    A = h.shape[0]
    nb = 4 * D * (A + 3 * E) + 4 * D * E + 4 * D * A * (2 if accumulate else 1) + 12 * A + 4 * (E + 1)
    with _timed("env_agg_bwd", dict(rows=A, segs=E, bytes=nb, saved_bytes=4 * D * E)):
        _lib.check(lib.matris_env_agg_bwd(h.shape[0], E, _p(h), _p(env), _p(g_agg), _p(S), _p(tgt.key), _p(src.key),
                                          _p(src.rowptr), _p(src.perm), int(accumulate), _p(g_h), _p(g_env),
                                          _stream()), "matris_env_agg_bwd")
    return g_env


# ------------------------------------------------------------------------------------
# fused gated MLP
# ------------------------------------------------------------------------------------
def pack_b(w, mode: int):
    """matris_pack_b of an fp32 [n, k] matrix whose rows are a GEMM's output columns."""
    w = _f32c(w)
    n, k = w.shape
    lib = _lib.load()
    out = torch.empty(lib.matris_pack_b_bytes(n, k, mode), dtype=torch.uint8, device=w.device)
    _lib.check(lib.matris_pack_b(n, k, _p(w), mode, _p(out), _stream()), "matris_pack_b")
    return out


class _PackCache:
    """fp32 weight matrices of one fused op, and their matris_pack_b images per MFMA mode,
    rebuilt when any source parameter changes (data pointer or version)."""

    def __init__(self):
        self.sig = None
        self.mats = {}
        self._packed = {}

    def _refresh(self, params, build):
        sig = tuple((p.data_ptr(), p._version, p.device) for p in params)
        if sig != self.sig:
            with torch.no_grad():
                build()
            self._packed = {}
            self.sig = sig

    def b(self, name: str, mode: int):
        key = (name, mode)
        if key not in self._packed:
            self._packed[key] = pack_b(self.mats[name], mode)
        return self._packed[key]


class GmlpPack(_PackCache):
    """GatedMLP weights: w1 = [core; gate] layer-0 weights [256, K], w2 = layer-3 weights
    [256, 128], their transposes for the backward, biases and norm weights."""

    def get(self, mod):
        params = (mod.mlp_core.layers[0].weight, mod.mlp_core.layers[0].bias, mod.mlp_core.layers[3].weight,
                  mod.mlp_core.layers[3].bias, mod.mlp_gate.layers[0].weight, mod.mlp_gate.layers[0].bias,
                  mod.mlp_gate.layers[3].weight, mod.mlp_gate.layers[3].bias, mod.core_norm.weight,
                  mod.gate_norm.weight)

        def build():
            c1w, c1b, c2w, c2b, g1w, g1b, g2w, g2b, nc, ng = (p.detach().float() for p in params)
            w1 = torch.cat([c1w, g1w], 0).contiguous()
            self.mats = {"w1": w1, "w2": torch.cat([c2w, g2w], 0).contiguous(), "w1t": w1.t().contiguous(),
                         "w2bt": torch.cat([c2w.t(), g2w.t()], 0).contiguous()}
            self.b1 = torch.cat([c1b, g1b], 0).contiguous()
            self.b2 = torch.cat([c2b, g2b], 0).contiguous()
            self.nc = nc.contiguous()
            self.ng = ng.contiguous()
            eps = mod.core_norm.eps
            self.eps = float(torch.finfo(torch.float32).eps if eps is None else eps)

        self._refresh(params, build)
        return self

    def get_tensors(self, w1, b1, w2, b2, norm_c, norm_g, eps: float):
        """The same pack from plain tensors: w1 [256, K] (core rows, then gate rows), b1
        [256] or None, w2 [256, 128] (core, then gate), b2 [256] or None, norm weights [128]."""
        params = tuple(t for t in (w1, b1, w2, b2, norm_c, norm_g) if t is not None)

        def build():
            W1, W2 = w1.detach().float().contiguous(), w2.detach().float().contiguous()
            self.mats = {"w1": W1, "w2": W2, "w1t": W1.t().contiguous(),
                         "w2bt": torch.cat([W2[:D].t(), W2[D:].t()], 0).contiguous()}
            z = torch.zeros(256, dtype=torch.float32, device=w1.device)
            self.b1 = (b1.detach().float() if b1 is not None else z).contiguous()
            self.b2 = (b2.detach().float() if b2 is not None else z).contiguous()
            self.nc = norm_c.detach().float().contiguous()
            self.ng = norm_g.detach().float().contiguous()

        self._refresh(params, build)
        self.eps = float(eps)
        return self

    def b_blocks(self, blocks: tuple, mode: int):
        """Pack of W1's column blocks `blocks` side by side ([256, 128 len(blocks)]): the
        layer-1 weight of the sources multiplied in place."""
        key = ("w1_cols", blocks, mode)
        if key not in self._packed:
            w1 = self.mats["w1"]
            self._packed[key] = pack_b(torch.cat([w1[:, D * j:D * (j + 1)] for j in blocks], 1).contiguous(), mode)
        return self._packed[key]

    def b_stack(self, blocks: tuple, mode: int):
        """Pack of W1's column blocks `blocks` stacked ([256 len(blocks), 128]): the weight
        of matris_gmlp_project for sources multiplied before their gather."""
        key = ("w1_stack", blocks, mode)
        if key not in self._packed:
            w1 = self.mats["w1"]
            self._packed[key] = pack_b(torch.cat([w1[:, D * j:D * (j + 1)] for j in blocks], 0).contiguous(), mode)
        return self._packed[key]


def _vec(w):
    """A [1, 128] residual weight as a contiguous fp32 [128] device vector."""
    return w.detach().reshape(-1).float().contiguous()


# Discarded saves: inside the original pass of a non-reentrant activation checkpoint the
# tensors a layer saves for its backward are dropped (the backward recomputes them), so
# the GatedMLP and FFN forwards there leave their saved pre-activations unwritten: p and z
# come back as uninitialised tensors of the right shape (the checkpoint still checks the
# shapes of what the recomputation saves against them) and the kernels skip those stores.
_DISCARD = {"on": False}


class discard_saves:
    """Context manager for the original pass of a checkpointed region (torch.utils.checkpoint
    context_fn): saved-for-backward activations are not written.  Everything a layer returns
    is computed as usual."""

    def __enter__(self):
        self.old = _DISCARD["on"]
        _DISCARD["on"] = True

    def __exit__(self, *exc):
        _DISCARD["on"] = self.old


# Gather after GEMM: in a GatedMLP of at least 2^16 rows, a gathered source whose table
# has at most a quarter as many rows is multiplied by its block of W1 once per table row
# (matris_gmlp_project) and its products are gathered instead of its features.  Measured
# at C3 (one box, whole step): the angle rows' bond and atom tables gain 0.8 ms, the
# edge rows' atom tables ~0.05 ms; projecting the edge rows' bond table (half as many
# rows as the layer) loses 0.15 ms, and smaller layers lose to the extra launch.
_GTG = {"on": True, "min_rows": 1 << 16, "ratio": 4}


class gather_after_gemm:
    """Context manager: switch the gather-after-GEMM forward of the GatedMLPs on or off,
    optionally with another threshold (layers of at least min_rows rows; tables of at
    most n_rows / ratio rows)."""

    def __init__(self, on: bool, min_rows: int | None = None, ratio: int | None = None):
        self.new = {"on": bool(on)}
        if min_rows is not None:
            self.new["min_rows"] = int(min_rows)
        if ratio is not None:
            self.new["ratio"] = int(ratio)

    def __enter__(self):
        self.old = dict(_GTG)
        _GTG.update(self.new)

    def __exit__(self, *exc):
        _GTG.update(self.old)


def _projected_sources(srcs, idxs, n_rows: int):
    """Indices of the sources to multiply before their gather (at most three)."""
    if not _GTG["on"] or n_rows < _GTG["min_rows"]:
        return []
    r = _GTG["ratio"]
    return [j for j, (s, i) in enumerate(zip(srcs, idxs)) if i is not None and r * s.shape[0] <= n_rows][:3]


def _gmlp_fwd_bytes(srcs, idxs, n_rows: int, saved: bool, res: bool, proj_tables=()) -> int:
    """Algorithmic HBM bytes of one GatedMLP forward launch: every input table read once
    (a gathered source's whole table, not its gathered rows; a projected source's product
    table), one int32 index per row and gathered source, out written once, p and z when
    saved, the residual source read and the residual output written."""
    b = 0
    for s, i in zip(srcs, idxs):
        b += 4 * D * (s.shape[0] if i is not None else n_rows) + (4 * n_rows if i is not None else 0)
    for rows, cols, n_idx in proj_tables:
        b += 4 * rows * cols + 4 * n_rows * n_idx
    return b + 4 * D * n_rows + (2 * 4 * 256 * n_rows if saved else 0) + (2 * 4 * D * n_rows if res else 0)


def gmlp_fwd_raw(pack: GmlpPack, srcs, idxs, n_rows: int, mode: int, res=None, save: bool = True):
    """matris_gmlp_fwd; srcs are [*,128] fp32 tensors, idxs int32 gather keys or None.
    res = (res_src, res_w) also returns res_out = out + res_w * res_src.
    Returns (out, p, z, res_out); the same whether or not sources are projected first
    (matris_gmlp_fwd_proj), up to the order of the fp32 sums of layer 1."""
    return _gmlp_fwd(pack, srcs, idxs, n_rows, mode, res, save, None)[:4]


def gmlp_fwd_ffn_raw(pack: GmlpPack, srcs, idxs, n_rows: int, mode: int, ffn: "_WeightPack", ffn_res=None,
                     ffn_res_w=None, save: bool = True):
    """matris_gmlp_fwd_ffn: the GatedMLP forward with the FFN tail on its output rows,
    ffn_out = W2 SiLU(W1 out) (+ ffn_res_w * ffn_res when given; ffn = the FFN's pack, as
    for ffn_fwd_raw).  Returns (out, p, z, ffn_out, ffn_p); p, z, ffn_p None when not
    saved."""
    out, p, z, _, t_out, t_p = _gmlp_fwd(pack, srcs, idxs, n_rows, mode, None, save, (ffn, ffn_res, ffn_res_w))
    return out, p, z, t_out, t_p


def gmlp_fwd_pair_raw(pack: GmlpPack, srcs, idxs, n_rows: int, mode: int, res, pair: "_WeightPack",
                      save: bool = True):
    """matris_gmlp_fwd_pair: gmlp_fwd_raw with res = (res_src, res_w) and the projection
    pair on res_src's rows in the same launch.  Returns (out, p, z, res_out, o0, o1) with
    (o0, o1) = pair_fwd_raw(pair, res_src)."""
    if res is None:
        raise ValueError("gmlp_fwd_pair_raw: the pair projects the residual source; res is required")
    return _gmlp_fwd(pack, srcs, idxs, n_rows, mode, res, save, None, pair)


def _gmlp_fwd(pack: GmlpPack, srcs, idxs, n_rows: int, mode: int, res, save: bool, tail, pair=None):
    lib = _lib.load()
    dev = srcs[0].device
    nsrc = len(srcs)
    # the kernel reads each source as [rows, 128] rows and W1 as 128-column blocks, one per
    # source: widths it cannot see through the pointers
    K = int(pack.mats["w1"].shape[1])
    if K != D * nsrc or any(s.dim() != 2 or s.shape[1] != D for s in srcs):
        raise ValueError(f"matris_gmlp_fwd: {nsrc} source(s) of shapes {[tuple(s.shape) for s in srcs]} for a "
                         f"layer-1 weight with K = {K}; each source must be [rows, 128] and K = 128 x sources")
    if any(i is None and s.shape[0] != n_rows for s, i in zip(srcs, idxs)):
        raise ValueError(f"matris_gmlp_fwd: an ungathered source must have the output's {n_rows} rows")
    out = _rows(n_rows, D, dev)
    p = _rows(n_rows, 256, dev) if save else None
    z = _rows(n_rows, 256, dev) if save else None
    res_out = _rows(n_rows, D, dev) if res is not None else None
    rs, rw = (res if res is not None else (None, None))
    proj = _projected_sources(srcs, idxs, n_rows)
    ret_p, ret_z = p, z
    t_out = t_p = ret_tp = None
    if tail is not None:
        t_pack, t_res, t_rw = tail
        if res is not None or (t_res is not None and (tuple(t_res.shape) != (n_rows, D) or not t_res.is_contiguous()
                                                      or t_rw is None)):
            raise ValueError("gmlp_fwd_ffn_raw: the residual source must be a contiguous [n_rows, 128] tensor, "
                             "with its weights")
        t_out = _rows(n_rows, D, dev)
        t_p = ret_tp = _rows(n_rows, D, dev) if save else None
    if _DISCARD["on"]:  # placeholders: the kernel writes neither
        p = z = t_p = None
    t_bytes = 0 if tail is None else 4 * D * n_rows * (1 + (t_res is not None) + (t_p is not None))
    if pair is not None:
        rs = _f32c(rs)
        if tuple(rs.shape) != (n_rows, D):
            raise ValueError("gmlp_fwd_pair_raw: the residual source must be [n_rows, 128]")
        t_out, ret_tp = _rows(n_rows, D, dev), _rows(n_rows, D, dev)
        t_bytes = 2 * 4 * D * n_rows  # the two projections written (res_src is read for res_out already)
    if tail is not None:
        # the tail rides the gather-after-GEMM entry point (with or without projected sources)
        t_args = (_p(t_pack.b("w0", mode)), _p(t_pack.b("w1", mode)), _p(t_p), _p(t_res),
                  _p(_f32c(t_rw) if t_rw is not None else None), _p(t_out))
    if not proj and tail is None and pair is None:
        src_arr = (ctypes.c_void_p * 4)(*[s.data_ptr() for s in srcs])
        idx_arr = (ctypes.c_void_p * 4)(*[(i.data_ptr() if i is not None else None) for i in idxs])
        with _timed("gmlp_fwd", dict(rows=n_rows, k=nsrc * D, extra_rows=0,
                                     bytes=_gmlp_fwd_bytes(srcs, idxs, n_rows, p is not None, res is not None),
                                     saved_bytes=2 * 4 * 256 * n_rows if p is not None else 0)):
            _lib.check(lib.matris_gmlp_fwd(n_rows, nsrc, src_arr, idx_arr, _p(pack.b("w1", mode)), _p(pack.b1),
                                           _p(pack.b("w2", mode)), _p(pack.b2), _p(pack.nc), _p(pack.ng), pack.eps,
                                           _p(out), _p(p), _p(z), _p(rs), _p(rw), _p(res_out), mode, _stream()),
                       "matris_gmlp_fwd")
        return out, ret_p, ret_z, res_out, None, None
    # one projection launch per distinct table, all of its blocks side by side (none when
    # nothing is projected: the FFN-tail launch with every source gathered)
    tables: dict = {}
    for j in proj:
        tables.setdefault((srcs[j].data_ptr(), srcs[j].shape[0]), []).append(j)
    p_ptr, p_idx, p_ld, keep = [], [], [], []
    for blocks in tables.values():
        x = srcs[blocks[0]]
        nb = len(blocks)
        P = _rows(x.shape[0], 256 * nb, dev)
        keep.append(P)
        with _timed("gmlp_proj", (x.shape[0], nb)):
            _lib.check(lib.matris_gmlp_project(x.shape[0], _p(x), _p(pack.b_stack(tuple(blocks), mode)), nb, _p(P),
                                               mode, _stream()), "matris_gmlp_project")
        for b, j in enumerate(blocks):
            p_ptr.append(P.data_ptr() + 4 * 256 * b)
            p_idx.append(idxs[j].data_ptr())
            p_ld.append(256 * nb)
    rest = [j for j in range(nsrc) if j not in proj]
    src_arr = (ctypes.c_void_p * 4)(*[srcs[j].data_ptr() for j in rest])
    idx_arr = (ctypes.c_void_p * 4)(*[(idxs[j].data_ptr() if idxs[j] is not None else None) for j in rest])
    n_pj = len(p_ptr)
    pj_arr = (ctypes.c_void_p * 3)(*p_ptr)
    pji_arr = (ctypes.c_void_p * 3)(*p_idx)
    pld_arr = (ctypes.c_int64 * 3)(*p_ld)
    w1 = _p(pack.b_blocks(tuple(rest), mode)) if rest else None
    ptab = [(keep[k].shape[0], keep[k].shape[1], len(b)) for k, b in enumerate(tables.values())]
    nbytes = _gmlp_fwd_bytes([srcs[j] for j in rest], [idxs[j] for j in rest], n_rows, p is not None,
                             res is not None, ptab) + t_bytes
    # k: the layer-1 width this kernel multiplies; extra_rows: rows of the FFN tail or the
    # projection pair (both add 2 * 128 * 256 FLOPs per row); saved_bytes: the pre-activations
    # written only for the backward (p, z and the tail's t), inside bytes
    saved = (2 * 4 * 256 * n_rows if p is not None else 0) + (4 * D * n_rows if t_p is not None and tail is not None
                                                                else 0)
    with _timed("gmlp_fwd", dict(rows=n_rows, k=len(rest) * D, bytes=nbytes, saved_bytes=saved,
                                 extra_rows=n_rows if (tail is not None or pair is not None) else 0)):
        if pair is not None:
            _lib.check(lib.matris_gmlp_fwd_pair(n_rows, len(rest), src_arr, idx_arr, n_pj, pj_arr, pji_arr, pld_arr,
                                                w1, _p(pack.b1), _p(pack.b("w2", mode)), _p(pack.b2), _p(pack.nc),
                                                _p(pack.ng), pack.eps, _p(out), _p(p), _p(z), _p(rs), _p(rw),
                                                _p(res_out), _p(pair.b("cat", mode)), _p(t_out), _p(ret_tp), mode,
                                                _stream()), "matris_gmlp_fwd_pair")
        elif tail is None:
            _lib.check(lib.matris_gmlp_fwd_proj(n_rows, len(rest), src_arr, idx_arr, n_pj, pj_arr, pji_arr, pld_arr,
                                                w1, _p(pack.b1), _p(pack.b("w2", mode)), _p(pack.b2), _p(pack.nc),
                                                _p(pack.ng), pack.eps, _p(out), _p(p), _p(z), _p(rs), _p(rw),
                                                _p(res_out), mode, _stream()), "matris_gmlp_fwd_proj")
        else:
            _lib.check(lib.matris_gmlp_fwd_ffn(n_rows, len(rest), src_arr, idx_arr, n_pj, pj_arr, pji_arr, pld_arr,
                                               w1, _p(pack.b1), _p(pack.b("w2", mode)), _p(pack.b2), _p(pack.nc),
                                               _p(pack.ng), pack.eps, _p(out), _p(p), _p(z), *t_args, mode,
                                               _stream()), "matris_gmlp_fwd_ffn")
    del keep  # the stream orders any later reuse of these blocks after the launch
    return out, ret_p, ret_z, res_out, t_out, ret_tp


def gmlp_tile_rows() -> int:
    """Rows per GatedMLP work-group tile (the tile of matris_gmlp_bwd_runs's partials)."""
    return int(_lib.load().matris_gmlp_tile_rows())


def gmlp_bwd_raw(pack: GmlpPack, g, p, z, K: int, mode: int, g_x=None, g_x0=None, acc0: bool = False, res_w=None,
                 runs=None, res_src=None, pair=None):
    """matris_gmlp_bwd.  Without g_x0 returns g_x [M, K]; with g_x0 source 0's gradient
    goes (accumulated if acc0, plus res_w * g if res_w) to g_x0 and the other columns to
    g_x [M, K-128] (allocated when not given; None when K == 128).
    runs = (key, blk): source block blk, gathered through `key` (int32 [M], ascending),
    leaves as tile-run partial sums (matris_gmlp_bwd_runs), to be completed by
    seg_sum_raw(..., tile_rows=gmlp_tile_rows()).  res_src: the residual term is
    res_w * res_src instead of res_w * g.  pair = (pack, g0, g1): g_x0 also gains
    pair_bwd_raw(pack, g0, g1) (matris_gmlp_bwd_pair; two-plane modes, with g_x0)."""
    lib = _lib.load()
    M = p.shape[0]
    if g_x is None and not (g_x0 is not None and K == D):
        g_x = _rows(M, K - (D if g_x0 is not None else 0), g.device)
    # algorithmic bytes: g_out, p, z (and the accumulated source-0 block) read once, g_x
    # written once; a run-summed block: its key read, at least one partial row per tile
    nbytes = 4 * M * (D + 2 * 256 + (D if (g_x0 is not None and acc0) else 0) + K + (D if res_src is not None else 0))
    if runs is not None:
        nbytes += 4 * M - 4 * D * M + 4 * D * -(-M // gmlp_tile_rows())
    if pair is not None:
        if mode == 6 or g_x0 is None or acc0:
            raise ValueError("gmlp_bwd_raw: pair needs a two-plane mode and a separate g_x0 (not accumulated)")
        pp, g0, g1 = pair
        for t in (g0, g1):
            if tuple(t.shape) != (M, D) or not t.is_contiguous():
                raise ValueError("gmlp_bwd_raw: pair gradients must be contiguous [M, 128] tensors")
        nbytes += 2 * 4 * D * M
        key, blk = runs if runs is not None else (None, -1)
        with _timed("gmlp_bwd", dict(rows=M, k=K, bytes=nbytes, saved_bytes=2 * 4 * 256 * M, extra_rows=M)):
            _lib.check(lib.matris_gmlp_bwd_pair(M, K, _p(g), _p(p), _p(z), _p(pack.b("w1t", mode)),
                                                _p(pack.b("w2bt", mode)), _p(pack.nc), _p(pack.ng), pack.eps, _p(g_x),
                                                _p(g_x0), _p(res_w), _p(res_src), _p(key), int(blk), _p(g0), _p(g1),
                                                _p(pp.b("cat_t", mode)), mode, _stream()), "matris_gmlp_bwd_pair")
        return g_x
    with _timed("gmlp_bwd", dict(rows=M, k=K, bytes=nbytes, saved_bytes=2 * 4 * 256 * M, extra_rows=0)):
        args = (M, K, _p(g), _p(p), _p(z), _p(pack.b("w1t", mode)), _p(pack.b("w2bt", mode)), _p(pack.nc),
                _p(pack.ng), pack.eps, _p(g_x), _p(g_x0), int(acc0), _p(res_w))
        if runs is None and res_src is None:
            _lib.check(lib.matris_gmlp_bwd(*args, mode, _stream()), "matris_gmlp_bwd")
        else:
            key, blk = runs if runs is not None else (None, -1)
            if key is not None and (key.dtype != torch.int32 or key.numel() != M or not key.is_contiguous()):
                raise ValueError("gmlp_bwd_raw: runs key must be a contiguous int32 tensor of one entry per row")
            if res_src is not None and (res_w is None or tuple(res_src.shape) != (M, D) or not res_src.is_contiguous()):
                raise ValueError("gmlp_bwd_raw: res_src must be a contiguous [M, 128] tensor, with res_w")
            _lib.check(lib.matris_gmlp_bwd_runs(*args, _p(res_src), _p(key), int(blk), mode, _stream()),
                       "matris_gmlp_bwd_runs")
    return g_x


def gmlp_bwd_ffn_raw(pack: GmlpPack, p, z, K: int, mode: int, ffn: "_WeightPack", ffn_g, ffn_p, env_term=None,
                     g_x0=None, res_w=None, runs=None, ffn_g_idx=None, ffn_g_scale: float = 1.0):
    """matris_gmlp_bwd_ffn: gmlp_bwd_raw(pack, g, p, z, K, mode, g_x0=g_x0, res_w=res_w,
    res_src=ffn_g, runs=runs) with g = ffn_bwd_raw(ffn, G, ffn_p, mode, env_term=...)
    computed inside the kernel (two-plane modes), G = ffn_g, or ffn_g_scale *
    ffn_g[ffn_g_idx] with an index (int32, one per row; not with res_w).  env_term =
    (ge, env, a, b): the term ge[a.key] * env[b.key] (a, b groupings with one key per row).
    Returns g_x as gmlp_bwd_raw does."""
    lib = _lib.load()
    M = p.shape[0]
    if mode == 6:
        raise ValueError("gmlp_bwd_ffn_raw: two-plane modes only (0, 2, 3)")
    if ffn_g_idx is None:
        if tuple(ffn_g.shape) != (M, D) or not ffn_g.is_contiguous():
            raise ValueError("gmlp_bwd_ffn_raw: ffn_g must be a contiguous [M, 128] tensor")
    elif (ffn_g_idx.dtype != torch.int32 or ffn_g_idx.numel() != M or not ffn_g_idx.is_contiguous()
          or ffn_g.shape[1] != D or not ffn_g.is_contiguous() or res_w is not None):
        raise ValueError("gmlp_bwd_ffn_raw: ffn_g_idx is one int32 row of ffn_g per row, without res_w")
    if tuple(ffn_p.shape) != (M, D) or not ffn_p.is_contiguous():
        raise ValueError("gmlp_bwd_ffn_raw: ffn_p must be a contiguous [M, 128] tensor")
    g_x = None if (g_x0 is not None and K == D) else _rows(M, K - (D if g_x0 is not None else 0), p.device)
    ge = env = tk = sk = None
    nbytes = 4 * M * (2 * D + 2 * 256 + K) if ffn_g_idx is None else \
        4 * M * (D + 2 * 256 + K + 1) + 4 * D * ffn_g.shape[0]
    if env_term is not None:
        ge, env, tgt, src = env_term
        tk, sk = tgt.key, src.key
        if tk.numel() != M or sk.numel() != M or ge.shape[1] != D or env.shape[1] != D:
            raise ValueError("gmlp_bwd_ffn_raw: env_term needs one key per row in both groupings, 128-wide tables")
        nbytes += 8 * M + 4 * D * (ge.shape[0] + env.shape[0])
    key, blk = runs if runs is not None else (None, -1)
    if key is not None:
        if key.dtype != torch.int32 or key.numel() != M or not key.is_contiguous():
            raise ValueError("gmlp_bwd_ffn_raw: runs key must be a contiguous int32 tensor of one entry per row")
        nbytes += 4 * M - 4 * D * M + 4 * D * -(-M // gmlp_tile_rows())
    # extra_rows: rows of the FFN head; saved_bytes: p, z and the FFN's pre-activation read
    with _timed("gmlp_bwd", dict(rows=M, k=K, bytes=nbytes, saved_bytes=4 * M * (2 * 256 + D), extra_rows=M)):
        _lib.check(lib.matris_gmlp_bwd_ffn(M, K, _p(p), _p(z), _p(pack.b("w1t", mode)), _p(pack.b("w2bt", mode)),
                                           _p(pack.nc), _p(pack.ng), pack.eps, _p(g_x), _p(g_x0), _p(res_w),
                                           _p(key), int(blk), _p(ffn_g), _p(ffn_g_idx), float(ffn_g_scale),
                                           _p(ffn_p), _p(ffn.b("wt0", mode)),
                                           _p(ffn.b("wt1", mode)), _p(ge), _p(env), _p(tk), _p(sk), mode, _stream()),
                   "matris_gmlp_bwd_ffn")
    return g_x


class _GatedMLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pack, groupings, n_rows, *srcs):
        _check_dev(*srcs)
        srcs = [_f32c(s) for s in srcs]
        mode = _MMA["mode"]
        out, p, z, _ = gmlp_fwd_raw(pack, srcs, [g.key if g is not None else None for g in groupings], n_rows, mode)
        ctx.mode = mode
        ctx.save_for_backward(p, z)
        ctx.pack, ctx.groupings = pack, groupings
        ctx.src_rows = [s.shape[0] for s in srcs]
        return out

    @staticmethod
    def backward(ctx, g):
        p, z = ctx.saved_tensors
        g = _f32c(g)
        K = D * len(ctx.groupings)
        g_x = gmlp_bwd_raw(ctx.pack, g, p, z, K, ctx.mode)
        grads = []
        for j, grp in enumerate(ctx.groupings):
            if not ctx.needs_input_grad[3 + j]:
                grads.append(None)
            elif grp is None:
                grads.append(g_x[:, j * D:(j + 1) * D])
            else:
                out = _rows(ctx.src_rows[j], D, g.device)
                seg_sum_raw(g_x, grp, 1.0, ldx=K, col_off=j * D, out=out)
                grads.append(out)
        return (None, None, None, *grads)


def gated_mlp(module, pack: GmlpPack, sources):
    """GatedMLP(cat_j src_j[idx_j]) fused on MFMA.  sources: list of (tensor, Grouping|None);
    a Grouping's key is the gather index, its CSR serves the backward scatter."""
    groupings = [g for _, g in sources]
    first = sources[0]
    n_rows = first[1].n_rows if first[1] is not None else first[0].shape[0]
    return _GatedMLP.apply(pack.get(module), groupings, n_rows, *[t for t, _ in sources])


# ------------------------------------------------------------------------------------
# dense layers on MFMA: FFN (Linear -> SiLU -> Linear, no bias) and the projection pair
# ------------------------------------------------------------------------------------
class _WeightPack(_PackCache):
    """Bias-free 128x128 Linear weights W0, W1 (FFN layers, or the W_s / W_t pair):
    mats w0, w1, their transposes wt0, wt1, and cat = [W0; W1], cat_t = cat^T."""

    def get(self, *params):
        def build():
            w = [p.detach().float().contiguous() for p in params]
            self.mats = {f"w{i}": t for i, t in enumerate(w)}
            self.mats.update({f"wt{i}": t.t().contiguous() for i, t in enumerate(w)})
            if len(w) > 1:
                cat = torch.cat(w, 0).contiguous()
                self.mats.update({"cat": cat, "cat_t": cat.t().contiguous()})

        self._refresh(params, build)
        self.device = params[0].device
        return self


def ffn_fwd_raw(pack: _WeightPack, x, mode: int, res=None, save: bool = True):
    """(out, p) of matris_ffn_fwd; res = (res_src, res_w) adds res_w * res_src to out;
    p (the saved pre-activation) is None when not saved."""
    lib = _lib.load()
    M = x.shape[0]
    out = _rows(M, D, x.device)
    p = _rows(M, D, x.device) if save else None
    rs, rw = (res if res is not None else (None, None))
    kp = None if _DISCARD["on"] else p  # discarded saves: a placeholder, not written
    with _timed("ffn_fwd", (M,)):
        _lib.check(lib.matris_ffn_fwd(M, _p(x), _p(pack.b("w0", mode)), _p(pack.b("w1", mode)), _p(out), _p(kp),
                                      _p(rs), _p(rw), mode, _stream()), "matris_ffn_fwd")
    return out, p


def ffn_bwd_raw(pack: _WeightPack, g, p, mode: int, g_res=None, res_w=None, env_term=None):
    """g_x of matris_ffn_bwd; g_res (given) receives res_w * g.  env_term = (g_agg_env, env,
    tgt, src): g_x also gains g_agg_env[tgt.key] * env[src.key] (matris_ffn_bwd_env)."""
    lib = _lib.load()
    M = p.shape[0]
    g_x = _rows(M, D, g.device)
    with _timed("ffn_bwd", (M,)):
        if env_term is None:
            _lib.check(lib.matris_ffn_bwd(M, _p(g), _p(p), _p(pack.b("wt0", mode)), _p(pack.b("wt1", mode)),
                                          _p(g_x), _p(g_res), _p(res_w), mode, _stream()), "matris_ffn_bwd")
        else:
            if g_res is not None:
                raise ValueError("ffn_bwd_raw: env_term and g_res do not combine")
            ge, env, tgt, src = env_term
            if tgt.key.numel() != M or src.key.numel() != M or ge.shape != env.shape:
                raise ValueError("ffn_bwd_raw: env_term needs one target / source per row and ge shaped as env")
            _lib.check(lib.matris_ffn_bwd_env(M, _p(g), _p(p), _p(pack.b("wt0", mode)), _p(pack.b("wt1", mode)),
                                              _p(g_x), _p(ge), _p(env), _p(tgt.key), _p(src.key), mode, _stream()),
                       "matris_ffn_bwd_env")
    return g_x


def pair_fwd_raw(pack: _WeightPack, x, mode: int):
    """(x W0^T, x W1^T) of matris_pair_fwd."""
    lib = _lib.load()
    M = x.shape[0]
    o0, o1 = _rows(M, D, x.device), _rows(M, D, x.device)
    with _timed("pair_fwd", (M,)):
        _lib.check(lib.matris_pair_fwd(M, _p(x), _p(pack.b("cat", mode)), _p(o0), _p(o1), mode, _stream()),
                   "matris_pair_fwd")
    return o0, o1


def pair_bwd_raw(pack: _WeightPack, g0, g1, mode: int, res=None, res_w=None, out=None, accumulate: bool = False):
    """g0 W0 + g1 W1 (+ res_w * res) of matris_pair_bwd, into `out` (allocated when None;
    its previous contents added last when accumulate)."""
    lib = _lib.load()
    M = g0.shape[0]
    if accumulate and out is None:
        raise ValueError("pair_bwd_raw: accumulate needs out")
    g_x = _rows(M, D, g0.device) if out is None else out
    with _timed("pair_bwd", (M,)):
        _lib.check(lib.matris_pair_bwd(M, _p(g0), _p(g1), _p(pack.b("cat_t", mode)), _p(g_x), _p(res), _p(res_w),
                                       int(accumulate), mode, _stream()), "matris_pair_bwd")
    return g_x


class _FFN(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, pack):
        _check_dev(x)
        x = _f32c(x)
        mode = _MMA["mode"]
        out, p = ffn_fwd_raw(pack, x, mode)
        ctx.save_for_backward(p)
        ctx.pack, ctx.mode = pack, mode
        return out

    @staticmethod
    def backward(ctx, g):
        (p,) = ctx.saved_tensors
        return ffn_bwd_raw(ctx.pack, _f32c(g), p, ctx.mode), None


def ffn(pack: _WeightPack, x):
    """W2 SiLU(W1 x) for an MLP(hidden=int, bias=False) (functions.py:198-205)."""
    return _FFN.apply(x, pack)


class _Pair(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, pack):
        _check_dev(x)
        x = _f32c(x)
        mode = _MMA["mode"]
        ctx.pack, ctx.mode = pack, mode
        return pair_fwd_raw(pack, x, mode)

    @staticmethod
    def backward(ctx, g0, g1):
        dev = ctx.pack.device
        ref = g0 if g0 is not None else g1
        M = ref.shape[0]
        g0 = _rows(M, D, dev).zero_() if g0 is None else _f32c(g0)
        g1 = _rows(M, D, dev).zero_() if g1 is None else _f32c(g1)
        return pair_bwd_raw(ctx.pack, g0, g1, ctx.mode), None


def proj_pair(pack: _WeightPack, x):
    """(x W0^T, x W1^T) for two bias-free 128x128 Linears in one MFMA pass."""
    return _Pair.apply(x, pack)


# ------------------------------------------------------------------------------------
# basis functions of the embeddings (E2, E3)
# ------------------------------------------------------------------------------------
class _Bessel(torch.autograd.Function):
    @staticmethod
    def forward(ctx, dist, freq, cutoff: float, p: float):
        _check_dev(dist, freq)
        dist, freq = _f32c(dist), _f32c(freq.detach())
        lib = _lib.load()
        n, nr = dist.shape[0], freq.shape[0]
        out = torch.empty(n, nr, device=dist.device)
        with _timed("bessel_fwd", (n,)):
            _lib.check(lib.matris_bessel_fwd(n, nr, _p(dist), _p(freq), cutoff, p, _p(out), _stream()),
                       "matris_bessel_fwd")
        ctx.save_for_backward(dist, freq)
        ctx.cutoff, ctx.p = cutoff, p
        return out

    @staticmethod
    def backward(ctx, g):
        dist, freq = ctx.saved_tensors
        lib = _lib.load()
        g = _f32c(g)
        g_dist = torch.empty_like(dist)
        with _timed("bessel_bwd", (dist.shape[0],)):
            _lib.check(lib.matris_bessel_bwd(dist.shape[0], freq.shape[0], _p(dist), _p(freq), ctx.cutoff, ctx.p,
                                             _p(g), 0, _p(g_dist), _stream()), "matris_bessel_bwd")
        return g_dist, None, None, None


def bessel(dist, freq, cutoff: float, envelope_exponent: float):
    """[n, len(freq)] Bessel basis times the polynomial envelope (basis_function.py:8-50,
    116-186); the backward returns the distance gradient only."""
    return _Bessel.apply(dist, freq, float(cutoff), float(envelope_exponent))


class _EdgeEmbed(torch.autograd.Function):
    """matris_edge_embed_fwd / _bwd: EdgeBasisEmbedding (feature_embed.py:42-148) per bond,
    differentiable in the edge lengths only (the efsm path takes no weight gradients)."""

    @staticmethod
    def forward(ctx, length, u2d32, mod):
        _check_dev(length, u2d32)
        length = _f32c(length)
        lib = _lib.load()
        mode = _MMA["mode"]
        b6, b4 = mod.pairwise_rbf_expansion, mod.threebody_rbf_expansion
        f6, f4 = _f32c(b6.frequencies.detach()), _f32c(b4.frequencies.detach())
        w1 = _f32c(mod.edge_linear1.weight.detach())
        ln = mod.edge_init_norm
        lg, lb = _f32c(ln.weight.detach()), _f32c(ln.bias.detach())
        pack = mod._pack.get(mod.edge_linear2.weight, mod.swish_layer.linear.weight)
        U, nr, dev = u2d32.shape[0], f6.shape[0], length.device
        e, h3, xhat = _rows(U, D, dev), _rows(U, D, dev), _rows(U, D, dev)
        rbf6, rbf4 = torch.empty(U, nr, device=dev), torch.empty(U, nr, device=dev)
        rstd = torch.empty(U, device=dev)
        args = (U, _p(length), _p(u2d32), _p(f6), float(b6.envelope_func.cutoff), _p(f4),
                float(b4.envelope_func.cutoff), nr, float(b6.envelope_func.p), _p(w1))
        with _timed("edge_embed_fwd", (U,)):
            _lib.check(lib.matris_edge_embed_fwd(*args, _p(pack.b("w0", mode)), _p(lg), _p(lb), float(ln.eps),
                                                 _p(pack.b("w1", mode)), _p(e), _p(rbf6), _p(rbf4), _p(h3), _p(xhat),
                                                 _p(rstd), mode, _stream()), "matris_edge_embed_fwd")
        ctx.save_for_backward(length, u2d32, f6, f4, w1, lg, h3, xhat, rstd)
        ctx.mod, ctx.mode, ctx.pack = mod, mode, pack
        ctx.set_materialize_grads(False)
        return e, rbf6, rbf4

    @staticmethod
    def backward(ctx, g_e, g6, g4):
        length, u2d32, f6, f4, w1, lg, h3, xhat, rstd = ctx.saved_tensors
        mod, mode, pack = ctx.mod, ctx.mode, ctx.pack
        U, dev = u2d32.shape[0], length.device
        g_len = torch.zeros_like(length)
        g_e = _zeros_if_none(g_e, h3)
        b6, b4 = mod.pairwise_rbf_expansion, mod.threebody_rbf_expansion
        with _timed("edge_embed_bwd", (U,)):
            _lib.check(_lib.load().matris_edge_embed_bwd(
                U, _p(length), _p(u2d32), _p(f6), float(b6.envelope_func.cutoff), _p(f4),
                float(b4.envelope_func.cutoff), f6.shape[0], float(b6.envelope_func.p), _p(w1),
                _p(pack.b("wt0", mode)), _p(lg), _p(pack.b("wt1", mode)), _p(g_e),
                _p(None if g6 is None else _f32c(g6)), _p(None if g4 is None else _f32c(g4)), _p(h3), _p(xhat),
                _p(rstd), _p(g_len), mode, _stream()), "matris_edge_embed_bwd")
        return g_len, None, None


def _zeros_if_none(g, like):
    return torch.zeros_like(like) if g is None else _f32c(g)


def edge_embed(length, u2d32, mod):
    """(e [U,128], rbf6 [U,7], rbf4 [U,7]) of EdgeBasisEmbedding `mod` for the bonds whose
    first directed edge is u2d32 (int32 [U]), from the directed edges' lengths [E]."""
    return _EdgeEmbed.apply(length, u2d32, mod)


class _SBF(torch.autograd.Function):
    @staticmethod
    def forward(ctx, unit, grp_t: Grouping, grp_s: Grouping, cutoff: float):
        _check_dev(unit)
        unit = _f32c(unit)
        lib = _lib.load()
        A = grp_t.n_rows
        out = _rows(A, 16, unit.device)
        with _timed("sbf_fwd", (A,)):
            _lib.check(lib.matris_sbf_fwd(A, _p(unit), _p(grp_t.key), _p(grp_s.key), cutoff, _p(out), _stream()),
                       "matris_sbf_fwd")
        ctx.save_for_backward(unit)
        ctx.grp_t, ctx.grp_s, ctx.cutoff = grp_t, grp_s, cutoff
        return out

    @staticmethod
    def backward(ctx, g):
        (unit,) = ctx.saved_tensors
        gt, gs = ctx.grp_t, ctx.grp_s
        lib = _lib.load()
        g = _f32c(g)
        g_unit = torch.empty_like(unit)
        A = gt.n_rows
        work = _rows(max(A, 1), 6, unit.device)
        with _timed("sbf_bwd", (unit.shape[0],)):
            _lib.check(lib.matris_sbf_bwd(unit.shape[0], A, _p(unit), _p(gt.key), _p(gs.key), _p(g), _p(gt.rowptr),
                                          _p(gt.perm), _p(gs.rowptr), _p(gs.perm), ctx.cutoff, 0, _p(work),
                                          _p(g_unit), _stream()), "matris_sbf_bwd")
        return g_unit, None, None, None


class _TbEmbed(torch.autograd.Function):
    """tb = SiLU(Ws (Wa b)) over the [A, 16] angle basis (matris_tb_embed_fwd / _bwd);
    input gradient only."""

    @staticmethod
    def forward(ctx, basis, wa, pack, mode):
        _check_dev(basis)
        lib = _lib.load()
        basis = _f32c(basis)
        M = basis.shape[0]
        out = _rows(M, D, basis.device)
        with _timed("tb_embed_fwd", (M,)):
            _lib.check(lib.matris_tb_embed_fwd(M, _p(basis), _p(wa), _p(pack.b("w0", mode)), _p(out), mode,
                                               _stream()), "matris_tb_embed_fwd")
        ctx.save_for_backward(basis)
        ctx.wa, ctx.pack, ctx.mode = wa, pack, mode
        return out

    @staticmethod
    def backward(ctx, g):
        (basis,) = ctx.saved_tensors
        lib = _lib.load()
        g = _f32c(g)
        M = basis.shape[0]
        g_b = torch.empty_like(basis)
        with _timed("tb_embed_bwd", (M,)):
            _lib.check(lib.matris_tb_embed_bwd(M, _p(basis), _p(g), _p(ctx.wa), _p(ctx.pack.b("w0", ctx.mode)),
                                               _p(ctx.pack.b("wt0", ctx.mode)), _p(g_b), ctx.mode, _stream()),
                       "matris_tb_embed_bwd")
        return g_b, None, None, None


def tb_embed_supported() -> bool:
    """The fused three-body embedding runs in the two-plane MFMA modes (fp32, f16x3, bf16x3)."""
    return _MMA["mode"] in (0, 2, 3)


def tb_embed(basis, wa_param, ws_param, pack: "_WeightPack"):
    """SiLU(ws (wa basis)) for bias-free Linear weights wa [128, 16], ws [128, 128]."""
    pack.get(ws_param)
    wa = wa_param.detach().float().contiguous()
    return _TbEmbed.apply(basis, wa, pack, _MMA["mode"])


def spherical_basis(unit, grp_t: Grouping, grp_s: Grouping, cutoff: float):
    """[A, 16] three-body basis of every angle from the unit edge vectors [E_d, 3]: grp_t /
    grp_s group the angles by the directed edge they read as i->j (target_DE_index) and
    j->k (source_DE_index) (feature_embed.py:183-201, basis_function.py:222-338)."""
    return _SBF.apply(unit, grp_t, grp_s, float(cutoff))


# ------------------------------------------------------------------------------------
# readout
# ------------------------------------------------------------------------------------
class ReadoutPack(_PackCache):
    """The readout's weights (RMSNorm weight, energy MLP 128-128-128-1, magmom MLP 128-256-1)
    in the layouts matris_readout_fwd / _bwd read, rebuilt when a parameter changes."""

    def get(self, norm, energy_mlp, magmom_mlp):
        L, M = energy_mlp.layers, magmom_mlp.layers
        lin_e = [l for l in L if isinstance(l, torch.nn.Linear)]
        lin_m = [l for l in M if isinstance(l, torch.nn.Linear)]
        params = (norm.weight, *[p for l in lin_e + lin_m for p in (l.weight, l.bias)])

        def build():
            w1, w2, w3 = (l.weight.detach().float() for l in lin_e)
            w4, w5 = (l.weight.detach().float() for l in lin_m)
            self.mats = dict(wn=norm.weight.detach().float().contiguous(), w1=w1.contiguous(),
                             w1t=w1.t().contiguous(), w2=w2.contiguous(), w2t=w2.t().contiguous(),
                             w3=w3.reshape(-1).contiguous(), w4t=w4.t().contiguous(),
                             w5=w5.reshape(-1).contiguous())
            for k, l in zip(("b1", "b2", "b3"), lin_e):
                self.mats[k] = l.bias.detach().float().reshape(-1).contiguous()
            for k, l in zip(("b4", "b5"), lin_m):
                self.mats[k] = l.bias.detach().float().reshape(-1).contiguous()
            eps = norm.eps
            self.eps = float(torch.finfo(torch.float32).eps if eps is None else eps)

        self._refresh(params, build)
        return self


def readout_fwd_raw(pack: ReadoutPack, x):
    """(e [N], m [N]) of matris_readout_fwd: per-row energy and |magmom| of the readout."""
    lib = _lib.load()
    x = _f32c(x)
    N = x.shape[0]
    e = torch.empty(N, dtype=torch.float32, device=x.device)
    m = torch.empty(N, dtype=torch.float32, device=x.device)
    w = pack.mats
    with _timed("readout_fwd", dict(rows=N)):
        _lib.check(lib.matris_readout_fwd(N, _p(x), _p(w["wn"]), _p(w["w1t"]), _p(w["b1"]), _p(w["w2t"]),
                                          _p(w["b2"]), _p(w["w3"]), _p(w["b3"]), _p(w["w4t"]), _p(w["b4"]),
                                          _p(w["w5"]), _p(w["b5"]), pack.eps, _p(e), _p(m), _stream()),
                   "matris_readout_fwd")
    return e, m


def readout_bwd_raw(pack: ReadoutPack, x, g_e):
    """g_x [N, 128] of matris_readout_bwd: the energy branch's input gradient."""
    lib = _lib.load()
    x, g_e = _f32c(x), _f32c(g_e)
    g_x = _rows(x.shape[0], D, x.device)
    w = pack.mats
    with _timed("readout_bwd", dict(rows=x.shape[0])):
        _lib.check(lib.matris_readout_bwd(x.shape[0], _p(x), _p(w["wn"]), _p(w["w1t"]), _p(w["b1"]), _p(w["w1"]),
                                          _p(w["w2t"]), _p(w["b2"]), _p(w["w2"]), _p(w["w3"]), pack.eps, _p(g_e),
                                          0, _p(g_x), _stream()), "matris_readout_bwd")
    return g_x


class Readout(torch.autograd.Function):
    """(e [N], m [N]) of the fused readout; e is differentiable (its backward is
    readout_bwd_raw), m is not (the magmom head is evaluated, never differentiated)."""

    @staticmethod
    def forward(ctx, x, pack):
        _check_dev(x)
        e, m = readout_fwd_raw(pack, x)
        ctx.save_for_backward(x)
        ctx.pack = pack
        ctx.mark_non_differentiable(m)
        return e, m

    @staticmethod
    def backward(ctx, g_e, g_m):
        (x,) = ctx.saved_tensors
        if g_e is None:
            return None, None
        return readout_bwd_raw(ctx.pack, x, g_e), None
